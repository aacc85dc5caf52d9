// Fused bf16 decode kernels for a Qwen2-style decoder layer on gfx950: skinny weight-streaming
// MFMA GEMMs (skinny.h) with fused prologues and epilogues. Rounding points are those of the
// unfused dli.graph.v1 graph (every op rounds its output to bf16), so fused and unfused graphs
// compute the same values up to fp32 summation order. A decoder layer is five launches: qkv,
// attention (attention.hip), o_proj, gate_up, down.
//
//  qkv_rope_append         [optional RMSNorm of x in registers] -> [q|k|v] = xn W^T + b ->
//                          interleaved RoPE on q, k (rotary/kernel.py:6-35) -> k, v written into
//                          the paged KV cache at each row's position, q out
//  linear_residual         out = residual + bf16(x W^T + b)          (one workgroup per 16 rows)
//  linear_residual_splitk  the same with K split over workgroups; the last split to finish a
//                          tile sums the partials (agent-scope stores/loads, arrival counter)
//  linear_partial          fp32 split-K partial tiles of x W^T: grid (N / 16, splits);
//  residual_rms_norm       h = bf16(residual + bf16(sum_s partial_s + b)) and
//                          xn = bf16(h * rsqrt(mean(h^2) + eps) * w) (rms_norm/kernel.py:6-14)
//  gate_up_silu            [optional RMSNorm of x in registers] -> gate/up = xn W^T ->
//                          bf16(bf16(silu(gate)) * up) (weights interleaved in 16-row blocks:
//                          [gate 16 rows | up 16 rows] per output block of 16)
//  lm_head_argmax          [optional final RMSNorm of x in registers] -> logits = xn W^T
//                          (fp32) -> logits out + per-workgroup argmax partials; argmax_finalize
//                          reduces them (first index of the maximum)
// qkv_rope_append, gate_up_silu and lm_head_argmax walk their weight tiles grid-strided
// (tileLoop), sized by the host to the workgroups that are resident at once, so the weight
// stream never waits on a second dispatch round.
#include "decode_parts.h"
#include "scratch.h"

using namespace dk;

// Device scratch of dli_hip_lm_head_argmax_norm_noalloc (the argmax partials that the
// other lm_head entry points keep in a caller's workspace), for callers that cannot allocate.
// One copy per device that loads this module, zero at load, held until the process ends. Its
// name stays in the code object's symbol table (no `static`), because the host finds it with
// hipModuleGetGlobal on the loaded module; host code only ever uses the address that lookup
// returns.
__device__ __align__(256) unsigned char scratch[dli_scratch::kLmHeadBytes];

namespace {

constexpr int kThreads = 256;
constexpr int kWaves = kThreads / kWave;
constexpr int kNormPer = 4;          // residual_rms_norm: N <= kThreads * kNormPer
constexpr int kMaxNormSplits = kMaxSplits;  // residual_rms_norm: split-K partials summed

// One 16-row weight tile per workgroup (72 workgroups for Qwen2-0.5B's 1152 q|k|v rows): the
// grid covers the tiles exactly, so the epilogue operands of tile blockIdx.x are prefetched.
// x is the residual stream, RMS-normalized in registers when norm_w is non-NULL.
template <int MB>
__device__ void qkv_rope_append_impl(const uint16_t* x, const uint16_t* norm_w, float eps,
                                     const uint16_t* w, const QkvParams& p, int K) {
  using Core = SkinnyCore<1, MB, kNormWaves, kNormUnroll>;
  __shared__ float lds[Core::kLdsFloats + kNormLdsFloats<MB, kNormWaves>];
  const int64_t N = static_cast<int64_t>(p.Hq + 2 * p.Hkv) * p.D;
  const int64_t n0 = static_cast<int64_t>(blockIdx.x) * Core::kTileN;
  QkvEpilogue<MB, PlainMem> epi;
  epi.prefetch(p, n0);  // epilogue operands do not depend on the GEMM: fetched first
  tileLoop<1, MB, kNormWaves, kNormUnroll>(w, XGlobal{x, K}, N, K, p.M, lds, norm_w, eps,
                                           blockIdx.x, gridDim.x, INT64_MAX, NoWait{},
                                           [&](int64_t) { epi.apply(p, n0, lds); });
}

// out = residual + bf16(x W^T + b); 16 weight rows per workgroup, 8 waves split K.
template <int MB>
__device__ void linear_residual_impl(const uint16_t* x, const uint16_t* w, const uint16_t* bias,
                                     const uint16_t* residual, uint16_t* out, int M, int64_t N,
                                     int K) {
  using Core = SkinnyCore<1, MB, kResWaves, (MB >= 4 ? 2 : 4)>;  // 256 VGPRs at 512 threads
  __shared__ float lds[Core::kLdsFloats];
  const int64_t n0 = static_cast<int64_t>(blockIdx.x) * Core::kTileN;
  ResidualTile<MB, kResThreads, PlainMem> rt;
  rt.load(residual, bias, n0, M, N);  // residual and bias fetched before the weights
  Core::run(w, XGlobal{x, K}, N, K, M, n0, 0, K / 64, lds);
  rt.store(out, n0, M, N, [&](int e) { return lds[e]; });
}

// out = residual + bf16(x W^T + b) with K split over grid.y (16 weight rows, 8 waves per
// workgroup): every split stores its partial tile and arrives at counters[tile]; the last split
// to arrive sums the partials in split order, writes the output tile and resets the counter to
// zero (splitKArrive). No cross-workgroup fence and no second kernel. splits <= kMaxSplits.
//   partials: [tiles][splits][16 x 16 MB] fp32, counters: [tiles] (zero before the first call)
template <int MB>
__device__ void linear_residual_splitk_impl(const uint16_t* x, const uint16_t* w,
                                            const uint16_t* bias, const uint16_t* residual,
                                            uint16_t* out, int M, int64_t N, int K, int splits,
                                            float* partials, unsigned* counters) {
  using Core = SkinnyCore<1, MB, kResWaves, 2, kDownIdle>;  // the decoder stack's down_proj core
  constexpr int kElems = Core::kTileN * Core::kTileM;
  __shared__ float lds[Core::kLdsFloats];
  __shared__ int is_last;
  const int64_t n0 = static_cast<int64_t>(blockIdx.x) * Core::kTileN;
  ResidualTile<MB, kResThreads, PlainMem> rt;
  rt.load(residual, bias, n0, M, N);  // residual and bias fetched before the weights
  int sb, se;
  splitRange(K / 64, blockIdx.y, splits, sb, se);
  Core::run(w, XGlobal{x, K}, N, K, M, n0, sb, se, lds);
  splitKArrive<MB, kResThreads, PlainMem>(
      lds, partials + static_cast<int64_t>(blockIdx.x) * splits * kElems, blockIdx.y, splits,
      counters + blockIdx.x, static_cast<unsigned>(splits), true, rt, out, n0, M, N, &is_last);
}

// partials[split][m][n] = sum over the split's K steps of x[m, k] * w[n, k]; 16 rows per
// workgroup.
template <int MB>
__device__ void linear_partial_impl(const uint16_t* x, const uint16_t* w, float* partials, int M,
                                    int64_t N, int K, int splits) {
  using Core = SkinnyCore<1, MB, kWaves>;
  __shared__ float lds[Core::kLdsFloats];
  const int64_t n0 = static_cast<int64_t>(blockIdx.x) * Core::kTileN;
  int sb, se;
  splitRange(K / 64, blockIdx.y, splits, sb, se);
  Core::run(w, XGlobal{x, K}, N, K, M, n0, sb, se, lds);
  float* dst = partials + static_cast<int64_t>(blockIdx.y) * M * N;
  for (int idx = threadIdx.x; idx < Core::kTileN * Core::kTileM; idx += kThreads) {
    const int nl = idx % Core::kTileN, m = idx / Core::kTileN;  // n fastest: coalesced stores
    const int64_t n = n0 + nl;
    if (m < M && n < N) dst[m * N + n] = lds[nl * Core::kTileM + m];
  }
}

// One workgroup per row m. With norm_w == nullptr only h is written. Every load of the row
// (residual, bias, norm weight and the partials of all splits, splits <= kMaxNormSplits) is
// issued before any is used, so their memory round trips overlap.
__device__ void residual_rms_norm_impl(const float* partials, int splits, const uint16_t* bias,
                                       const uint16_t* residual, const uint16_t* norm_w,
                                       uint16_t* h_out, uint16_t* xn_out, int M, int N, float eps) {
  __shared__ float scratch[kWaves];
  const int m = blockIdx.x;
  float part[kMaxNormSplits][kNormPer], hv[kNormPer], bv[kNormPer], wv[kNormPer];
#pragma unroll
  for (int j = 0; j < kNormPer; ++j) {
    const int n = threadIdx.x + j * kThreads;
    const bool ok = n < N;
    hv[j] = ok ? bf16ToFloat(residual[static_cast<int64_t>(m) * N + n]) : 0.f;
    bv[j] = ok && bias != nullptr ? bf16ToFloat(bias[n]) : 0.f;
    wv[j] = ok && norm_w != nullptr ? bf16ToFloat(norm_w[n]) : 0.f;
#pragma unroll
    for (int sp = 0; sp < kMaxNormSplits; ++sp)
      part[sp][j] = ok && sp < splits ? partials[(static_cast<int64_t>(sp) * M + m) * N + n] : 0.f;
  }
  float sq = 0.f;
#pragma unroll
  for (int j = 0; j < kNormPer; ++j) {
    const int n = threadIdx.x + j * kThreads;
    float y = part[0][j];
#pragma unroll
    for (int sp = 1; sp < kMaxNormSplits; ++sp) y += part[sp][j];  // split order; absent = +0
    y += bv[j];
    hv[j] = roundBf16(hv[j] + roundBf16(y));
    sq += hv[j] * hv[j];
    if (n < N) h_out[static_cast<int64_t>(m) * N + n] = floatToBf16(hv[j]);
  }
  if (norm_w == nullptr) return;
  const float inv = 1.0f / sqrtf(blockSum(sq, scratch) / static_cast<float>(N) + eps);
#pragma unroll
  for (int j = 0; j < kNormPer; ++j) {
    const int n = threadIdx.x + j * kThreads;
    if (n < N) xn_out[static_cast<int64_t>(m) * N + n] = floatToBf16(hv[j] * inv * wv[j]);
  }
}

// x is the residual stream, RMS-normalized in registers when norm_w is non-NULL.
template <int MB>
__device__ void gate_up_silu_impl(const uint16_t* x, const uint16_t* norm_w, float eps,
                                  const uint16_t* w_gu, uint16_t* out, int M, int64_t F, int K) {
  using Core = SkinnyCore<2, MB, kNormWaves, kNormUnroll>;
  __shared__ float lds[Core::kLdsFloats + kNormLdsFloats<MB, kNormWaves>];
  tileLoop<2, MB, kNormWaves, kNormUnroll, PlainMem, false, (MB >= 2)>(
      w_gu, XGlobal{x, K}, 2 * F, K, M, lds, norm_w, eps, blockIdx.x, gridDim.x, INT64_MAX, NoWait{},
      [&](int64_t t) { gateUpEpilogue<MB, PlainMem, (MB >= 2)>(lds, out, M, F, t); });
}

constexpr int kLmTileN = 32;  // vocab rows per lm_head tile (NF = 2)
constexpr int kLmQuarters = kLmTileN / 4;
constexpr int kLmStageTiles = 12;  // tiles of logits a workgroup holds in LDS before writing them

// Writes `staged` tiles of logits staged in LDS (slot j: tile first + j * stride, batch row m at
// m * kRow floats) to out [M, V] (float or bfloat16). A lane writes kPer consecutive logits of
// one row with one 16-byte store when `wide` (16-byte aligned rows) and the chunk lies inside
// the vocabulary; other chunks are written element by element.
template <bool kF32, int kTileM, int kTileN, int kRow, typename T>
__device__ __forceinline__ void flushStagedLogits(const float* stage, int staged, int64_t first,
                                                  int64_t stride, T* out, int M, int64_t V,
                                                  bool wide) {
  constexpr int kPer = kF32 ? 4 : 8;
  constexpr int kChunks = kTileN / kPer;  // per batch row of a tile
  for (int idx = threadIdx.x; idx < staged * kTileM * kChunks; idx += kThreads) {
    const int j = idx / (kTileM * kChunks), e = idx % (kTileM * kChunks);
    const int c = e % kChunks, m = e / kChunks;  // a row's chunks on adjacent lanes
    if (m >= M) continue;
    const int64_t n = (first + j * stride) * kTileN + c * kPer;
    const float* src = stage + j * kTileM * kRow + m * kRow + c * kPer;
    T* dst = out + static_cast<int64_t>(m) * V + n;
    if (wide && n + kPer <= V) {
      U128 o;
      if constexpr (kF32) {
#pragma unroll
        for (int i = 0; i < 4; ++i) o[i] = __builtin_bit_cast(uint32_t, src[i]);
      } else {
#pragma unroll
        for (int i = 0; i < 4; ++i) o[i] = packBf16x2(src[2 * i], src[2 * i + 1]);
      }
      PlainMem::store16(dst, o);
    } else {
      for (int i = 0; i < kPer && n + i < V; ++i) {
        if constexpr (kF32)
          dst[i] = src[i];
        else
          dst[i] = floatToBf16(src[i]);
      }
    }
  }
}

// Logits of vocab tiles of 32 rows (grid-strided over the workgroups) plus each workgroup's
// argmax partial per row, part_*[m * gridDim.x + blockIdx.x]: the first index of the largest
// logit among the workgroup's tiles. Requires K / 64 <= 4 * kWaves.
// With norm_w non-NULL, xn is the un-normalized residual stream and its final RMSNorm
// (model.norm, bf16 output) is applied in registers first (tileLoop's prologue).
//
// The tile loop issues no global store while its LDS staging has room: the tile logits are
// staged in LDS (fp32, rows padded to kTileN + 1 floats against bank conflicts) and written
// after the loop, or whenever kLmStageTiles tiles are staged, as 16-byte stores of 4 fp32 or
// 8 bf16 logits; the argmax runs in registers, one (row, quarter of the tile rows) item per
// thread, and is merged per workgroup once. At 32 rows, 896 columns and 151,936 vocabulary rows
// this takes the launch from 64 to 56 us against one 2-byte logit store per thread and tile
// plus per-tile argmax partials inside the loop.
template <int MB>
__device__ void lm_head_argmax_impl(const uint16_t* xn, const uint16_t* w, void* logits,
                                    int logits_f32, float* part_val, int32_t* part_idx, int M,
                                    int64_t V, int K, const uint16_t* norm_w, float eps) {
  using Core = SkinnyCore<2, MB, kWaves>;
  static_assert(Core::kTileN == kLmTileN, "lm_head tile");
  constexpr int kTileM = Core::kTileM, kTileN = Core::kTileN;
  constexpr int kRow = kTileN + 1;             // staged floats per batch row of a tile
  constexpr int kStageFloats = kTileM * kRow;  // per staged tile
  constexpr int kItems = (kLmQuarters * kTileM + kThreads - 1) / kThreads;
  // the tile reductions, then the staged logits (during the prologue only, the RMSNorm row sums)
  static_assert(kNormLdsFloats<MB, kWaves> <= kLmStageTiles * kStageFloats, "lm_head lds");
  static_assert(2 * kLmQuarters * kTileM <= Core::kLdsFloats, "lm_head quarter merge");
  __shared__ float lds[Core::kLdsFloats + kLmStageTiles * kStageFloats];
  float* const stage = lds + Core::kLdsFloats;
  const int64_t stride = gridDim.x;
  int64_t stage_first = blockIdx.x;  // tile of stage slot 0; slot j holds stage_first + j stride
  int staged = 0;
  // 16-byte stores (4 fp32 or 8 bf16 logits) wherever rows stay 16-byte aligned
  const bool wide = (reinterpret_cast<uintptr_t>(logits) & 15) == 0 && V % (logits_f32 ? 4 : 8) == 0;
  auto flush = [&]() {
    if (logits_f32)
      flushStagedLogits<true, kTileM, kTileN, kRow>(stage, staged, stage_first, stride,
                                                    static_cast<float*>(logits), M, V, wide);
    else
      flushStagedLogits<false, kTileM, kTileN, kRow>(stage, staged, stage_first, stride,
                                                     static_cast<uint16_t*>(logits), M, V, wide);
  };
  float best[kItems];
  int32_t arg[kItems];
#pragma unroll
  for (int i = 0; i < kItems; ++i) {
    best[i] = -INFINITY;
    arg[i] = -1;
  }
  tileLoop<2, MB, kWaves, 4>(w, XGlobal{xn, K}, V, K, M, lds, norm_w, eps, blockIdx.x, stride,
                             INT64_MAX, NoWait{}, [&](int64_t t) {
    const int64_t n0 = t * kTileN;
    if (logits != nullptr) {
      if (staged == kLmStageTiles) {
        flush();
        __syncthreads();  // every slot read before slot 0 is written again
        stage_first = t;
        staged = 0;
      }
      float* const slot = stage + staged * kStageFloats;
      for (int idx = threadIdx.x; idx < kTileN * kTileM; idx += kThreads) {
        const int m = idx % kTileM, nl = idx / kTileM;
        slot[m * kRow + nl] = lds[nl * kTileM + m];
      }
      ++staged;
    }
    // thread item (m, q) scans rows 4q..4q+3 of each tile in order: first index of the maximum
#pragma unroll
    for (int i = 0; i < kItems; ++i) {
      const int idx = threadIdx.x + i * kThreads;
      if (idx >= kLmQuarters * kTileM) break;
      const int m = idx % kTileM, q = idx / kTileM;
#pragma unroll
      for (int j = 0; j < 4; ++j) {
        const int nl = q * 4 + j;
        const float v = lds[nl * kTileM + m];
        if (n0 + nl < V && (arg[i] < 0 || v > best[i])) {
          best[i] = v;
          arg[i] = static_cast<int32_t>(n0 + nl);
        }
      }
    }
  });
  // tileLoop ends every tile with a barrier: the staging is complete and the reduction area free
  if (logits != nullptr) flush();
  float* const qv = lds;
  int32_t* const qa = reinterpret_cast<int32_t*>(lds + kLmQuarters * kTileM);
#pragma unroll
  for (int i = 0; i < kItems; ++i) {
    const int idx = threadIdx.x + i * kThreads;
    if (idx >= kLmQuarters * kTileM) break;
    qv[idx] = best[i];  // idx = q * kTileM + m
    qa[idx] = arg[i];
  }
  __syncthreads();
  for (int m = threadIdx.x; m < M; m += kThreads) {
    float b = -INFINITY;
    int32_t a = -1;
    for (int q = 0; q < kLmQuarters; ++q) {  // the quarters interleave: ties go to the lower index
      const float v = qv[q * kTileM + m];
      const int32_t i = qa[q * kTileM + m];
      if (i >= 0 && (a < 0 || v > b || (v == b && i < a))) {
        b = v;
        a = i;
      }
    }
    part_val[static_cast<int64_t>(m) * stride + blockIdx.x] = b;
    part_idx[static_cast<int64_t>(m) * stride + blockIdx.x] = a < 0 ? 0x7fffffff : a;
  }
}

// One workgroup per row: reduce that row's partials (contiguous, one per lm_head workgroup);
// ties keep the lower index.
__device__ void argmax_finalize_impl(const float* part_val, const int32_t* part_idx, int parts,
                                     int64_t* ids) {
  __shared__ float sv[kWaves];
  __shared__ int32_t si[kWaves];
  const int m = blockIdx.x;
  const float* vals = part_val + static_cast<int64_t>(m) * parts;
  const int32_t* idxs = part_idx + static_cast<int64_t>(m) * parts;
  float best = -INFINITY;
  int32_t arg = 0x7fffffff;
  constexpr int kBatch = 8;  // loads of kBatch partials in flight per thread
  for (int t0 = threadIdx.x; t0 < parts; t0 += kBatch * kThreads) {
    float v[kBatch];
    int32_t ix[kBatch];
#pragma unroll
    for (int u = 0; u < kBatch; ++u) {
      const int t = t0 + u * kThreads;
      v[u] = t < parts ? vals[t] : -INFINITY;
      ix[u] = t < parts ? idxs[t] : 0x7fffffff;
    }
#pragma unroll
    for (int u = 0; u < kBatch; ++u) {
      if (v[u] > best || (v[u] == best && ix[u] < arg)) {
        best = v[u];
        arg = ix[u];
      }
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

#define DK_DECODE_KERNELS(MB)                                                                     \
  extern "C" __global__ void __launch_bounds__(kNormThreads) qkv_rope_append_m##MB(               \
      const uint16_t* x, const uint16_t* norm_w, float eps, const uint16_t* w,                    \
      const uint16_t* bias, const float* cos_t, const float* sin_t, int64_t max_pos,              \
      const void* positions, int pos64, uint16_t* q_out, uint16_t* k_pool, uint16_t* v_pool,      \
      const int32_t* block_table, int64_t block_size, int64_t max_blocks, int M, int K, int Hq,   \
      int Hkv, int D) {                                                                           \
    const QkvParams p{bias, cos_t, sin_t, max_pos, positions, pos64, q_out,                       \
                      KvCacheArgs{k_pool, v_pool, block_table, block_size, max_blocks}, M, Hq,    \
                      Hkv, D};                                                                    \
    qkv_rope_append_impl<MB>(x, norm_w, eps, w, p, K);                                            \
  }                                                                                               \
  extern "C" __global__ void __launch_bounds__(kResWaves * 64) linear_residual_m##MB(             \
      const uint16_t* x, const uint16_t* w, const uint16_t* bias, const uint16_t* residual,       \
      uint16_t* out, int M, int64_t N, int K) {                                                   \
    linear_residual_impl<MB>(x, w, bias, residual, out, M, N, K);                                 \
  }                                                                                               \
  extern "C" __global__ void __launch_bounds__(kResThreads) linear_residual_splitk_m##MB(         \
      const uint16_t* x, const uint16_t* w, const uint16_t* bias, const uint16_t* residual,       \
      uint16_t* out, int M, int64_t N, int K, int splits, float* partials, unsigned* counters) {  \
    linear_residual_splitk_impl<MB>(x, w, bias, residual, out, M, N, K, splits, partials,         \
                                    counters);                                                    \
  }                                                                                               \
  extern "C" __global__ void __launch_bounds__(kThreads, MB >= 4 ? 1 : 2) linear_partial_m##MB(   \
      const uint16_t* x, const uint16_t* w, float* partials, int M, int64_t N, int K,             \
      int splits) {                                                                               \
    linear_partial_impl<MB>(x, w, partials, M, N, K, splits);                                     \
  }                                                                                               \
  extern "C" __global__ void __launch_bounds__(kNormThreads) gate_up_silu_m##MB(                  \
      const uint16_t* x, const uint16_t* norm_w, float eps, const uint16_t* w_gu, uint16_t* out,  \
      int M, int64_t F, int K) {                                                                  \
    gate_up_silu_impl<MB>(x, norm_w, eps, w_gu, out, M, F, K);                                    \
  }                                                                                               \
  extern "C" __global__ void __launch_bounds__(kThreads, MB >= 4 ? 1 : 2) lm_head_argmax_m##MB(    \
      const uint16_t* xn, const uint16_t* w, void* logits, int logits_f32, float* part_val,       \
      int32_t* part_idx, int M, int64_t V, int K, const uint16_t* norm_w, float eps) {            \
    lm_head_argmax_impl<MB>(xn, w, logits, logits_f32, part_val, part_idx, M, V, K, norm_w, eps); \
  }

DK_DECODE_KERNELS(1)
DK_DECODE_KERNELS(2)
DK_DECODE_KERNELS(4)

extern "C" __global__ void __launch_bounds__(kThreads)
    residual_rms_norm(const float* partials, int splits, const uint16_t* bias,
                      const uint16_t* residual, const uint16_t* norm_w, uint16_t* h_out,
                      uint16_t* xn_out, int M, int N, float eps) {
  residual_rms_norm_impl(partials, splits, bias, residual, norm_w, h_out, xn_out, M, N, eps);
}

extern "C" __global__ void __launch_bounds__(kThreads)
    argmax_finalize(const float* part_val, const int32_t* part_idx, int tiles, int64_t* ids) {
  argmax_finalize_impl(part_val, part_idx, tiles, ids);
}
