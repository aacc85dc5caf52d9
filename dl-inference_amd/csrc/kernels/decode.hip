// Fused bf16 decode kernels for a Qwen2-style decoder layer on gfx950. Each one is a skinny
// weight-streaming GEMM (skinny.h) with a fused prologue and/or epilogue. The rounding points
// are those of the unfused dli.graph.v1 graph (every op rounds its output to bf16), so the
// fused and unfused graphs compute the same values up to fp32 summation order:
//
//  qkv_rope_append   rms_norm -> [q|k|v] linear (+bias) -> interleaved RoPE on q, k
//                    (rotary/kernel.py:6-35) -> k, v scattered into the paged KV cache, q out
//  linear_residual   linear (+bias) -> add residual            (o_proj, down_proj)
//  gate_up_silu      rms_norm -> gate/up linear -> silu(gate) * up  (weights interleaved in
//                    16-row blocks: [gate 16 rows | up 16 rows] per output block of 16)
//  lm_head_argmax    rms_norm -> logits linear (fp32 accumulate) -> logits out + per-tile
//                    argmax partials; argmax_finalize reduces them (first index of the max)
//
// Launch: 256 threads, grid.x = N tiles of 32 weight rows, grid.y = K splits (split-K uses
// the last-arriving-workgroup reduction of skinny.h). Kernels taking an RMSNorm prologue
// keep the normalized activations in dynamic LDS ([16 * MB][K + 8] bf16).
#include "common.h"
#include "skinny.h"

using namespace dk;

namespace {

constexpr int kThreads = 256;
constexpr int kWaves = kThreads / kWave;
constexpr int kNormVec = 2;          // RMSNorm prologue: hidden <= 64 lanes * 8 * kNormVec = 1024
constexpr int kQkvNF = 1;            // qkv_rope_append: 16 weight rows per workgroup
constexpr int kResNF = 1;            // linear_residual: 16 weight rows per workgroup
constexpr int kResWaves = 8;         // linear_residual: 8 waves split K inside a workgroup
constexpr int kLmTilesPerBlock = 8;  // lm_head_argmax: 8 x 32 vocab rows per workgroup

// Steps [begin, end) of split `split` out of `splits` over `steps` 64-column steps.
__device__ __forceinline__ void splitRange(int steps, int split, int splits, int& begin, int& end) {
  const int per = (steps + splits - 1) / splits;
  begin = split * per;
  end = begin + per < steps ? begin + per : steps;
}

__device__ __forceinline__ float roundBf16(float v) { return bf16ToFloat(floatToBf16(v)); }

struct KvCacheArgs {
  uint16_t* k_pool;
  uint16_t* v_pool;
  const int32_t* block_table;
  int64_t block_size;
  int64_t max_blocks;
};

template <int MB>
__device__ void qkv_rope_append_impl(const uint16_t* h, const uint16_t* norm_w, const uint16_t* w,
                                     const uint16_t* bias, const float* cos_t, const float* sin_t,
                                     int64_t max_pos, const void* positions, int pos64,
                                     uint16_t* q_out, KvCacheArgs kv, int M, int K, int Hq, int Hkv,
                                     int D, float eps, float* partials, uint32_t* counters,
                                     int splits) {
  using Core = SkinnyCore<kQkvNF, MB, kWaves>;
  extern __shared__ __align__(16) unsigned char smem[];
  const int xstride = K + 8;
  uint16_t* xs = reinterpret_cast<uint16_t*>(smem);
  float* lds = reinterpret_cast<float*>(smem + Core::kTileM * xstride * sizeof(uint16_t));

  const int64_t N = static_cast<int64_t>(Hq + 2 * Hkv) * D;
  const int64_t n0 = static_cast<int64_t>(blockIdx.x) * Core::kTileN;
  const int64_t q_rows = static_cast<int64_t>(Hq) * D;
  const int64_t k_rows = static_cast<int64_t>(Hkv) * D;
  const int half = D / 2;
  const int64_t capacity = kv.max_blocks * kv.block_size;

  // Epilogue operands do not depend on the GEMM: fetch them first (position, then the rotary
  // coefficients, the bias pair and the cache block of this thread's (pair, row) items).
  constexpr int kItems = ((Core::kTileN / 2) * Core::kTileM + kThreads - 1) / kThreads;
  int64_t pos[kItems];
  float cs[kItems][2], bs[kItems][2];
  int64_t blk[kItems];
#pragma unroll
  for (int it = 0; it < kItems; ++it) {
    const int idx = threadIdx.x + it * kThreads;
    const int m = idx % Core::kTileM;
    pos[it] = (idx < (Core::kTileN / 2) * Core::kTileM && m < M) ? loadIndex(positions, pos64, m) : -1;
  }
#pragma unroll
  for (int it = 0; it < kItems; ++it) {
    const int idx = threadIdx.x + it * kThreads;
    const int pair = idx / Core::kTileM, m = idx % Core::kTileM;
    const int64_t n = n0 + 2 * pair;
    const bool live = pos[it] >= 0 && n < N;
    const int64_t local = n < q_rows ? n : (n < q_rows + k_rows ? n - q_rows : n - q_rows - k_rows);
    const int d = static_cast<int>(local % D);
    const bool rot = live && n < q_rows + k_rows && pos[it] < max_pos;
    cs[it][0] = rot ? cos_t[pos[it] * half + d / 2] : 1.f;
    cs[it][1] = rot ? sin_t[pos[it] * half + d / 2] : 0.f;
    bs[it][0] = (live && bias != nullptr) ? bf16ToFloat(bias[n]) : 0.f;
    bs[it][1] = (live && bias != nullptr) ? bf16ToFloat(bias[n + 1]) : 0.f;
    blk[it] = (live && n >= q_rows && pos[it] < capacity)
                  ? kv.block_table[m * kv.max_blocks + pos[it] / kv.block_size]
                  : -1;
  }

  int sb, se;
  splitRange(K / 64, blockIdx.y, splits, sb, se);
  Core::run(w, XLds{xs, xstride}, N, K, M, n0, sb, se, lds, [&] {
    rmsNormRowsToLds<Core::kTileM / kWaves, kNormVec>(h, norm_w, M, Core::kTileM, K, eps, xs, xstride);
  });
  if (!splitKReduce<Core::kTileN * Core::kTileM>(lds, partials, counters, blockIdx.x, blockIdx.y,
                                                   splits))
    return;

#pragma unroll
  for (int it = 0; it < kItems; ++it) {
    const int idx = threadIdx.x + it * kThreads;
    const int pair = idx / Core::kTileM;
    const int m = idx % Core::kTileM;
    const int64_t n = n0 + 2 * pair;
    if (pos[it] < 0 || n >= N) continue;
    // linear output (bias added, rounded), then the rotation in fp32, rounded again
    float v0 = roundBf16(lds[(2 * pair) * Core::kTileM + m] + bs[it][0]);
    float v1 = roundBf16(lds[(2 * pair + 1) * Core::kTileM + m] + bs[it][1]);
    const bool is_q = n < q_rows;
    const bool is_k = !is_q && n < q_rows + k_rows;
    const int64_t local = is_q ? n : (is_k ? n - q_rows : n - q_rows - k_rows);
    const int head = static_cast<int>(local / D);
    const int d = static_cast<int>(local % D);
    if (is_q || is_k) {
      const float r0 = v0 * cs[it][0] - v1 * cs[it][1];
      const float r1 = v0 * cs[it][1] + v1 * cs[it][0];
      v0 = r0;
      v1 = r1;
    }
    const uint16_t b0 = floatToBf16(v0), b1 = floatToBf16(v1);
    if (is_q) {
      uint16_t* dst = q_out + (static_cast<int64_t>(m) * Hq + head) * D + d;
      dst[0] = b0;
      dst[1] = b1;
      continue;
    }
    if (blk[it] < 0) continue;
    const int64_t off = pos[it] % kv.block_size;
    if (is_k) {
      uint16_t* dst = kv.k_pool + ((blk[it] * Hkv + head) * kv.block_size + off) * D + d;
      dst[0] = b0;
      dst[1] = b1;
    } else {
      uint16_t* dst = kv.v_pool + ((blk[it] * Hkv + head) * D + d) * kv.block_size + off;
      dst[0] = b0;
      dst[kv.block_size] = b1;
    }
  }
}

template <int MB>
__device__ void linear_residual_impl(const uint16_t* x, const uint16_t* w, const uint16_t* bias,
                                     const uint16_t* residual, uint16_t* out, int M, int64_t N,
                                     int K, float* partials, uint32_t* counters, int splits) {
  using Core = SkinnyCore<kResNF, MB, kResWaves>;
  __shared__ float lds[Core::kLdsFloats];
  const int64_t n0 = static_cast<int64_t>(blockIdx.x) * Core::kTileN;
  constexpr int kThreadsRes = kResWaves * kWave;
  constexpr int kItems = (Core::kTileN * Core::kTileM + kThreadsRes - 1) / kThreadsRes;
  float res[kItems];
#pragma unroll
  for (int it = 0; it < kItems; ++it) {  // residual (+ bias) fetched before the weights
    const int idx = threadIdx.x + it * kThreadsRes;
    const int nl = idx / Core::kTileM, m = idx % Core::kTileM;
    const int64_t n = n0 + nl;
    const bool live = idx < Core::kTileN * Core::kTileM && m < M && n < N;
    res[it] = live ? bf16ToFloat(residual[m * N + n]) : 0.f;
  }
  int sb, se;
  splitRange(K / 64, blockIdx.y, splits, sb, se);
  Core::run(w, XGlobal{x, K}, N, K, M, n0, sb, se, lds);
  if (!splitKReduce<Core::kTileN * Core::kTileM>(lds, partials, counters, blockIdx.x, blockIdx.y,
                                                   splits))
    return;
#pragma unroll
  for (int it = 0; it < kItems; ++it) {
    const int idx = threadIdx.x + it * kThreadsRes;
    const int nl = idx / Core::kTileM, m = idx % Core::kTileM;
    const int64_t n = n0 + nl;
    if (idx >= Core::kTileN * Core::kTileM || m >= M || n >= N) continue;
    float y = lds[idx];
    if (bias != nullptr) y += bf16ToFloat(bias[n]);
    y = roundBf16(y);
    out[m * N + n] = floatToBf16(res[it] + y);
  }
}

template <int MB>
__device__ void gate_up_silu_impl(const uint16_t* h, const uint16_t* norm_w, const uint16_t* w_gu,
                                  uint16_t* out, int M, int64_t F, int K, float eps) {
  using Core = SkinnyCore<2, MB, kWaves>;
  extern __shared__ __align__(16) unsigned char smem[];
  const int xstride = K + 8;
  uint16_t* xs = reinterpret_cast<uint16_t*>(smem);
  float* lds = reinterpret_cast<float*>(smem + Core::kTileM * xstride * sizeof(uint16_t));
  const int64_t n0 = static_cast<int64_t>(blockIdx.x) * Core::kTileN;  // rows of w_gu
  Core::run(w_gu, XLds{xs, xstride}, 2 * F, K, M, n0, 0, K / 64, lds, [&] {
    rmsNormRowsToLds<Core::kTileM / kWaves, kNormVec>(h, norm_w, M, Core::kTileM, K, eps, xs, xstride);
  });
  const int64_t f0 = static_cast<int64_t>(blockIdx.x) * 16;
  for (int idx = threadIdx.x; idx < 16 * Core::kTileM; idx += blockDim.x) {
    const int j = idx / Core::kTileM, m = idx % Core::kTileM;
    const int64_t f = f0 + j;
    if (m >= M || f >= F) continue;
    const float g = roundBf16(lds[j * Core::kTileM + m]);
    const float u = roundBf16(lds[(16 + j) * Core::kTileM + m]);
    const float s = roundBf16(g / (1.0f + expf(-g)));
    out[m * F + f] = floatToBf16(s * u);
  }
}

// Multiplies one vocab tile already loaded into `bt`, stores its logits and argmax partials.
template <int MB, typename Batch>
__device__ void lmHeadTile(Batch& bt, const XLds& xsrc, float* lds, void* logits, int logits_f32,
                           float* part_val, int32_t* part_idx, int M, int64_t V, int64_t t,
                           int steps, int r, int g, int wave) {
  using Core = SkinnyCore<2, MB, kWaves>;
  f32x4 acc[2][MB];
#pragma unroll
  for (int f = 0; f < 2; ++f)
#pragma unroll
    for (int b = 0; b < MB; ++b) acc[f][b] = f32x4{0.f, 0.f, 0.f, 0.f};
  Core::compute(acc, bt, xsrc, M, wave, steps, r, g);
  Core::reduce(acc, lds, r, g, wave);
  const int64_t n0 = t * Core::kTileN;
  if (logits != nullptr) {
    for (int idx = threadIdx.x; idx < Core::kTileN * Core::kTileM; idx += blockDim.x) {
      const int nl = idx / Core::kTileM, m = idx % Core::kTileM;
      const int64_t n = n0 + nl;
      if (m >= M || n >= V) continue;
      if (logits_f32)
        static_cast<float*>(logits)[m * V + n] = lds[idx];
      else
        static_cast<uint16_t*>(logits)[m * V + n] = floatToBf16(lds[idx]);
    }
  }
  // per-row argmax of this tile's fp32 logits (first index among equal maxima)
  for (int m = threadIdx.x; m < M; m += blockDim.x) {
    float best = -INFINITY;
    int32_t arg = static_cast<int32_t>(n0);
    for (int nl = 0; nl < Core::kTileN && n0 + nl < V; ++nl) {
      const float v = lds[nl * Core::kTileM + m];
      if (v > best) {
        best = v;
        arg = static_cast<int32_t>(n0 + nl);
      }
    }
    part_val[t * M + m] = best;
    part_idx[t * M + m] = arg;
  }
  __syncthreads();  // lds is reused by the next tile
}

// Vocab tiles of 32 rows; kLmTilesPerBlock consecutive tiles per workgroup share one normalized
// copy of x, and tile t + 1's weights stream in while tile t is multiplied. Requires
// K / 64 <= kUnroll * kWaves (one batch per tile).
template <int MB>
__device__ void lm_head_argmax_impl(const uint16_t* h, const uint16_t* norm_w, const uint16_t* w,
                                    void* logits, int logits_f32, float* part_val,
                                    int32_t* part_idx, int M, int64_t V, int K, float eps) {
  using Core = SkinnyCore<2, MB, kWaves>;
  using Batch = typename Core::template Batch<XLds>;
  extern __shared__ __align__(16) unsigned char smem[];
  const int xstride = K + 8;
  uint16_t* xs = reinterpret_cast<uint16_t*>(smem);
  float* lds = reinterpret_cast<float*>(smem + Core::kTileM * xstride * sizeof(uint16_t));
  const XLds xsrc{xs, xstride};
  const int lane = threadIdx.x % kWave, wave = threadIdx.x / kWave;
  const int r = lane % 16, g = lane / 16;
  const int steps = K / 64;
  const int64_t tiles = (V + Core::kTileN - 1) / Core::kTileN;
  const int64_t t_first = static_cast<int64_t>(blockIdx.x) * kLmTilesPerBlock;
  const int64_t t_last = t_first + kLmTilesPerBlock < tiles ? t_first + kLmTilesPerBlock : tiles;

  Batch bufA, bufB;
  Core::issue(bufA, Core::rows(w, V, K, t_first * Core::kTileN, r, g), xsrc, M, wave, steps, r, g);
  rmsNormRowsToLds<Core::kTileM / kWaves, kNormVec>(h, norm_w, M, Core::kTileM, K, eps, xs, xstride);
  for (int64_t t = t_first; t < t_last; t += 2) {
    if (t + 1 < t_last)
      Core::issue(bufB, Core::rows(w, V, K, (t + 1) * Core::kTileN, r, g), xsrc, M, wave, steps, r, g);
    lmHeadTile<MB>(bufA, xsrc, lds, logits, logits_f32, part_val, part_idx, M, V, t, steps, r, g, wave);
    if (t + 1 >= t_last) break;
    if (t + 2 < t_last)
      Core::issue(bufA, Core::rows(w, V, K, (t + 2) * Core::kTileN, r, g), xsrc, M, wave, steps, r, g);
    lmHeadTile<MB>(bufB, xsrc, lds, logits, logits_f32, part_val, part_idx, M, V, t + 1, steps, r, g,
                   wave);
  }
}

// One block per row: reduce tile partials in tile order (ties keep the lower index).
__device__ void argmax_finalize_impl(const float* part_val, const int32_t* part_idx, int tiles,
                                     int M, int64_t* ids) {
  __shared__ float sv[kWaves];
  __shared__ int32_t si[kWaves];
  const int m = blockIdx.x;
  float best = -INFINITY;
  int32_t arg = 0x7fffffff;
  for (int t = threadIdx.x; t < tiles; t += blockDim.x) {
    const float v = part_val[static_cast<int64_t>(t) * M + m];
    const int32_t i = part_idx[static_cast<int64_t>(t) * M + m];
    if (v > best || (v == best && i < arg)) {
      best = v;
      arg = i;
    }
  }
#pragma unroll
  for (int off = kWave / 2; off > 0; off >>= 1) {
    const float ov = __shfl_xor(best, off, kWave);
    const int32_t oi = __shfl_xor(arg, off, kWave);
    if (ov > best || (ov == best && oi < arg)) {
      best = ov;
      arg = oi;
    }
  }
  const int lane = threadIdx.x % kWave, wave = threadIdx.x / kWave;
  if (lane == 0) {
    sv[wave] = best;
    si[wave] = arg;
  }
  __syncthreads();
  if (threadIdx.x == 0) {
    for (int w = 1; w < kWaves; ++w) {
      if (sv[w] > best || (sv[w] == best && si[w] < arg)) {
        best = sv[w];
        arg = si[w];
      }
    }
    ids[m] = arg == 0x7fffffff ? 0 : arg;
  }
}

}  // namespace

#define DK_DECODE_KERNELS(MB)                                                                    \
  extern "C" __global__ void __launch_bounds__(kThreads) qkv_rope_append_m##MB(                  \
      const uint16_t* h, const uint16_t* norm_w, const uint16_t* w, const uint16_t* bias,        \
      const float* cos_t, const float* sin_t, int64_t max_pos, const void* positions, int pos64,  \
      uint16_t* q_out, uint16_t* k_pool, uint16_t* v_pool, const int32_t* block_table,           \
      int64_t block_size, int64_t max_blocks, int M, int K, int Hq, int Hkv, int D, float eps,   \
      float* partials, uint32_t* counters, int splits) {                                         \
    qkv_rope_append_impl<MB>(h, norm_w, w, bias, cos_t, sin_t, max_pos, positions, pos64, q_out, \
                             KvCacheArgs{k_pool, v_pool, block_table, block_size, max_blocks}, M, \
                             K, Hq, Hkv, D, eps, partials, counters, splits);                    \
  }                                                                                              \
  extern "C" __global__ void __launch_bounds__(kResWaves * 64) linear_residual_m##MB(                  \
      const uint16_t* x, const uint16_t* w, const uint16_t* bias, const uint16_t* residual,      \
      uint16_t* out, int M, int64_t N, int K, float* partials, uint32_t* counters, int splits) { \
    linear_residual_impl<MB>(x, w, bias, residual, out, M, N, K, partials, counters, splits);    \
  }                                                                                              \
  extern "C" __global__ void __launch_bounds__(kThreads) gate_up_silu_m##MB(                     \
      const uint16_t* h, const uint16_t* norm_w, const uint16_t* w_gu, uint16_t* out, int M,     \
      int64_t F, int K, float eps) {                                                             \
    gate_up_silu_impl<MB>(h, norm_w, w_gu, out, M, F, K, eps);                                   \
  }                                                                                              \
  extern "C" __global__ void __launch_bounds__(kThreads) lm_head_argmax_m##MB(                   \
      const uint16_t* h, const uint16_t* norm_w, const uint16_t* w, void* logits, int logits_f32, \
      float* part_val, int32_t* part_idx, int M, int64_t V, int K, float eps) {                  \
    lm_head_argmax_impl<MB>(h, norm_w, w, logits, logits_f32, part_val, part_idx, M, V, K, eps); \
  }

DK_DECODE_KERNELS(1)
DK_DECODE_KERNELS(2)
DK_DECODE_KERNELS(4)

extern "C" __global__ void __launch_bounds__(kThreads)
    argmax_finalize(const float* part_val, const int32_t* part_idx, int tiles, int M, int64_t* ids) {
  argmax_finalize_impl(part_val, part_idx, tiles, M, ids);
}
