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
//                          (fp32) -> logits out + per-tile argmax partials; argmax_finalize
//                          reduces them (first index of the maximum)
// qkv_rope_append, gate_up_silu and lm_head_argmax walk their weight tiles grid-strided
// (tileLoop), sized by the host to the workgroups that are resident at once, so the weight
// stream never waits on a second dispatch round.
#include "decode_parts.h"
#include "scratch.h"

using namespace dk;

// Device scratch of dli_hip_lm_head_argmax_norm_noalloc (the per-tile argmax partials that the
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
  using Core = SkinnyCore<1, MB, kResWaves, 2>;
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
  tileLoop<2, MB, kNormWaves, kNormUnroll>(
      w_gu, XGlobal{x, K}, 2 * F, K, M, lds, norm_w, eps, blockIdx.x, gridDim.x, INT64_MAX, NoWait{},
      [&](int64_t t) { gateUpEpilogue<MB, PlainMem>(lds, out, M, F, t); });
}

constexpr int kLmTileN = 32;  // vocab rows per lm_head tile (NF = 2)
constexpr int kLmQuarters = kLmTileN / 4;

// Logits of vocab tiles of 32 rows (grid-strided over the workgroups) plus each tile's argmax
// partial per row: part_*[m * tiles + t]. Requires K / 64 <= 4 * kWaves.
// With norm_w non-NULL, xn is the un-normalized residual stream and its final RMSNorm
// (model.norm, bf16 output) is applied in registers first (tileLoop's prologue).
template <int MB>
__device__ void lm_head_argmax_impl(const uint16_t* xn, const uint16_t* w, void* logits,
                                    int logits_f32, float* part_val, int32_t* part_idx, int M,
                                    int64_t V, int K, const uint16_t* norm_w, float eps) {
  using Core = SkinnyCore<2, MB, kWaves>;
  static_assert(Core::kTileN == kLmTileN, "lm_head tile");
  // the tile reductions, then the argmax quarters (inside the reductions' area) or, during the
  // prologue only, the RMSNorm row sums (after it)
  static_assert(kNormLdsFloats<MB, kWaves> <= kLmQuarters * Core::kTileM, "lm_head lds");
  __shared__ float lds[Core::kLdsFloats + kLmQuarters * Core::kTileM];
  __shared__ int lds_arg[kLmQuarters * Core::kTileM];
  const int64_t tiles = (V + Core::kTileN - 1) / Core::kTileN;
  tileLoop<2, MB, kWaves, 4>(w, XGlobal{xn, K}, V, K, M, lds, norm_w, eps, blockIdx.x,
                             gridDim.x, INT64_MAX, NoWait{}, [&](int64_t t) {
    const int64_t n0 = t * Core::kTileN;
    if (logits != nullptr) {
      for (int idx = threadIdx.x; idx < Core::kTileN * Core::kTileM; idx += kThreads) {
        const int nl = idx % Core::kTileN, m = idx / Core::kTileN;  // n fastest: coalesced stores
        const int64_t n = n0 + nl;
        if (m >= M || n >= V) continue;
        const float v = lds[nl * Core::kTileM + m];
        if (logits_f32)
          static_cast<float*>(logits)[m * V + n] = v;
        else
          static_cast<uint16_t*>(logits)[m * V + n] = floatToBf16(v);
      }
    }
    // argmax: thread (m, q) scans rows 4q..4q+3 of the tile, then one thread per m merges the
    // quarters in order (first index among equal maxima).
    float* qv = lds + Core::kTileN * Core::kTileM;
    for (int idx = threadIdx.x; idx < kLmQuarters * Core::kTileM; idx += kThreads) {
      const int m = idx % Core::kTileM, q = idx / Core::kTileM;
      float best = -INFINITY;
      int arg = -1;
#pragma unroll
      for (int j = 0; j < 4; ++j) {
        const int nl = q * 4 + j;
        const float v = lds[nl * Core::kTileM + m];
        if (n0 + nl < V && (arg < 0 || v > best)) {
          best = v;
          arg = nl;
        }
      }
      qv[q * Core::kTileM + m] = best;
      lds_arg[q * Core::kTileM + m] = arg;
    }
    __syncthreads();
    for (int m = threadIdx.x; m < M; m += kThreads) {
      float best = -INFINITY;
      int arg = -1;
      for (int q = 0; q < kLmQuarters; ++q) {
        const float v = qv[q * Core::kTileM + m];
        const int a = lds_arg[q * Core::kTileM + m];
        if (a >= 0 && (arg < 0 || v > best)) {
          best = v;
          arg = a;
        }
      }
      part_val[m * tiles + t] = best;
      part_idx[m * tiles + t] = static_cast<int32_t>(n0 + (arg < 0 ? 0 : arg));
    }
  });
}

// One workgroup per row: reduce that row's tile partials (contiguous) in tile order; ties keep
// the lower index.
__device__ void argmax_finalize_impl(const float* part_val, const int32_t* part_idx, int tiles,
                                     int64_t* ids) {
  __shared__ float sv[kWaves];
  __shared__ int32_t si[kWaves];
  const int m = blockIdx.x;
  const float* vals = part_val + static_cast<int64_t>(m) * tiles;
  const int32_t* idxs = part_idx + static_cast<int64_t>(m) * tiles;
  float best = -INFINITY;
  int32_t arg = 0x7fffffff;
  constexpr int kBatch = 8;  // loads of kBatch partials in flight per thread
  for (int t0 = threadIdx.x; t0 < tiles; t0 += kBatch * kThreads) {
    float v[kBatch];
    int32_t ix[kBatch];
#pragma unroll
    for (int u = 0; u < kBatch; ++u) {
      const int t = t0 + u * kThreads;
      v[u] = t < tiles ? vals[t] : -INFINITY;
      ix[u] = t < tiles ? idxs[t] : 0x7fffffff;
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
  extern "C" __global__ void __launch_bounds__(kThreads, 2) linear_partial_m##MB(                 \
      const uint16_t* x, const uint16_t* w, float* partials, int M, int64_t N, int K,             \
      int splits) {                                                                               \
    linear_partial_impl<MB>(x, w, partials, M, N, K, splits);                                     \
  }                                                                                               \
  extern "C" __global__ void __launch_bounds__(kNormThreads) gate_up_silu_m##MB(                  \
      const uint16_t* x, const uint16_t* norm_w, float eps, const uint16_t* w_gu, uint16_t* out,  \
      int M, int64_t F, int K) {                                                                  \
    gate_up_silu_impl<MB>(x, norm_w, eps, w_gu, out, M, F, K);                                    \
  }                                                                                               \
  extern "C" __global__ void __launch_bounds__(kThreads, 2) lm_head_argmax_m##MB(                  \
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
