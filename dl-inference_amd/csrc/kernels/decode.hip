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
//  lm_head_argmax          logits = xn W^T (fp32) -> logits out + per-tile argmax partials;
//                          argmax_finalize reduces them (first index of the maximum)
// qkv_rope_append, gate_up_silu and lm_head_argmax walk their weight tiles grid-strided
// (tileLoop), sized by the host to the workgroups that are resident at once, so the weight
// stream never waits on a second dispatch round.
#include "common.h"
#include "skinny.h"

using namespace dk;

namespace {

constexpr int kThreads = 256;
constexpr int kWaves = kThreads / kWave;
// qkv_rope_append and gate_up_silu (RMSNorm prologue): 8 waves, two per SIMD, so one wave's
// normalize VALU runs while the other is held issuing its weight loads.
constexpr int kNormWaves = 8;
constexpr int kNormThreads = kNormWaves * kWave;
constexpr int kNormUnroll = 2;  // 8 waves x 2 steps x 64 columns: hidden <= 1024
constexpr int kResWaves = 8;         // linear_residual: 8 waves split K inside a workgroup
constexpr int kNormPer = 4;          // residual_rms_norm: N <= kThreads * kNormPer
constexpr int kMaxNormSplits = 8;    // residual_rms_norm: split-K partials summed

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

// RMSNorm of x fragments held in registers, every 64-column step of K being in `xb` (lanes of
// wave w hold steps w, w + kW, ...): x[m, k] <- bf16(x[m, k] * rsqrt(mean_k x[m, k]^2 + eps)
// * w[k]) (rms_norm/kernel.py:6-14). Row sums of squares are reduced over the 4 lanes of a row
// and then over the waves through lds (kW * 16 * MB floats) in a fixed order.
template <int NF, int MB, int kW, int kU>
__device__ __forceinline__ void normalizeFragments(
    typename SkinnyCore<NF, MB, kW, kU>::XBatch& xb, const uint16_t* norm_w, int K, float eps,
    float* lds, int wave, int steps, int r, int g) {
  using Core = SkinnyCore<NF, MB, kW, kU>;
  U128 wv[kU][2];
#pragma unroll
  for (int u = 0; u < kU; ++u) {
    const int s = wave + u * kW;
    if (s >= steps) break;  // uniform: wave comes from readfirstlane
    const int64_t k0 = static_cast<int64_t>(s) * 64 + g * 8;
    wv[u][0] = load16(norm_w + k0);
    wv[u][1] = load16(norm_w + k0 + 32);
  }
  float sq[MB];
#pragma unroll
  for (int b = 0; b < MB; ++b) {
    sq[b] = 0.f;
#pragma unroll
    for (int u = 0; u < kU; ++u) {
      if (wave + u * kW >= steps) break;
#pragma unroll
      for (int h = 0; h < 2; ++h)
#pragma unroll
        for (int e = 0; e < 4; ++e) {
          const float lo = bf16ToFloat(static_cast<uint16_t>(xb.x[u][b][h][e]));
          const float hi = bf16ToFloat(static_cast<uint16_t>(xb.x[u][b][h][e] >> 16));
          sq[b] += lo * lo + hi * hi;
        }
    }
    sq[b] += __shfl_xor(sq[b], 16, kWave);
    sq[b] += __shfl_xor(sq[b], 32, kWave);
    if (g == 0) lds[wave * Core::kTileM + b * 16 + r] = sq[b];
  }
  __syncthreads();
  float inv[MB];
#pragma unroll
  for (int b = 0; b < MB; ++b) {
    float total = 0.f;
#pragma unroll
    for (int v = 0; v < kW; ++v) total += lds[v * Core::kTileM + b * 16 + r];
    inv[b] = 1.0f / sqrtf(total / static_cast<float>(K) + eps);
  }
  __syncthreads();  // lds is reused by the tile reductions
#pragma unroll
  for (int u = 0; u < kU; ++u) {
    if (wave + u * kW >= steps) break;
#pragma unroll
    for (int b = 0; b < MB; ++b)
#pragma unroll
      for (int h = 0; h < 2; ++h)
#pragma unroll
        for (int e = 0; e < 4; ++e) {
          const uint32_t xw = xb.x[u][b][h][e], ww = wv[u][h][e];
          const float lo = bf16ToFloat(static_cast<uint16_t>(xw)) * inv[b] *
                           bf16ToFloat(static_cast<uint16_t>(ww));
          const float hi = bf16ToFloat(static_cast<uint16_t>(xw >> 16)) * inv[b] *
                           bf16ToFloat(static_cast<uint16_t>(ww >> 16));
          xb.x[u][b][h][e] = packBf16x2(lo, hi);
        }
  }
}

// Weight tiles t = blockIdx.x, + gridDim.x, ... (16 * NF rows each) against one x whose
// fragments are loaded once (and RMS-normalized with norm_w when it is non-NULL) and stay in
// registers; the next tile's weights stream in while the current one is multiplied. epi(t)
// reads the reduced tile [16 NF][16 MB] from lds (row n, column m at lds[n * 16 MB + m]).
// Requires K / 64 <= kU * kW.
template <int NF, int MB, int kW, int kU, typename Epi>
__device__ __forceinline__ void tileLoop(const uint16_t* w, const XGlobal& xs, int64_t N, int K,
                                         int M, float* lds, const uint16_t* norm_w, float eps,
                                         Epi&& epi) {
  using Core = SkinnyCore<NF, MB, kW, kU>;
  const int lane = threadIdx.x % kWave;
  const int wave = __builtin_amdgcn_readfirstlane(threadIdx.x / kWave);
  const int r = lane % 16, g = lane / 16;
  const int steps = K / 64;
  const int64_t tiles = (N + Core::kTileN - 1) / Core::kTileN;
  const int64_t stride = gridDim.x;
  int64_t t = blockIdx.x;
  if (t >= tiles) return;
  typename Core::WBatch bufA, bufB;
  typename Core::XBatch xb;
  // x first: loads complete in issue order, so the RMSNorm of x (VALU) overlaps the weight
  // stream instead of waiting behind it. The second tile's weights are requested before the
  // prologue too.
  Core::issueX(xb, Core::xrows(xs, M, r, g), wave, steps);
  Core::issueW(bufA, Core::rows(w, N, K, t * Core::kTileN, r, g), wave, steps);
  if (t + stride < tiles)
    Core::issueW(bufB, Core::rows(w, N, K, (t + stride) * Core::kTileN, r, g), wave, steps);
  if (norm_w != nullptr)
    normalizeFragments<NF, MB, kW, kU>(xb, norm_w, K, eps, lds, wave, steps, r, g);
  auto tile = [&](const typename Core::WBatch& wb, int64_t tt) {
    f32x4 acc[NF][MB];
    Core::zero(acc);
    Core::compute(acc, wb, xb, wave, steps);
    Core::reduce(acc, lds, r, g, wave);
    epi(tt);
    __syncthreads();  // lds is reused by the next tile
  };
  for (bool first = true; t < tiles; t += 2 * stride, first = false) {
    if (!first && t + stride < tiles)
      Core::issueW(bufB, Core::rows(w, N, K, (t + stride) * Core::kTileN, r, g), wave, steps);
    tile(bufA, t);
    if (t + stride >= tiles) break;
    if (t + 2 * stride < tiles)
      Core::issueW(bufA, Core::rows(w, N, K, (t + 2 * stride) * Core::kTileN, r, g), wave, steps);
    tile(bufB, t + stride);
  }
}

// One 16-row weight tile per workgroup (72 workgroups for Qwen2-0.5B's 1152 q|k|v rows): the
// grid covers the tiles exactly, so the epilogue operands of tile blockIdx.x are prefetched.
// x is the residual stream, RMS-normalized in registers when norm_w is non-NULL.
template <int MB>
__device__ void qkv_rope_append_impl(const uint16_t* x, const uint16_t* norm_w, float eps,
                                     const uint16_t* w, const uint16_t* bias, const float* cos_t,
                                     const float* sin_t, int64_t max_pos, const void* positions,
                                     int pos64, uint16_t* q_out, KvCacheArgs kv, int M, int K,
                                     int Hq, int Hkv, int D) {
  using Core = SkinnyCore<1, MB, kNormWaves, kNormUnroll>;
  __shared__ float lds[Core::kLdsFloats];
  const int64_t N = static_cast<int64_t>(Hq + 2 * Hkv) * D;
  const int64_t n0 = static_cast<int64_t>(blockIdx.x) * Core::kTileN;
  const int64_t q_rows = static_cast<int64_t>(Hq) * D;
  const int64_t k_rows = static_cast<int64_t>(Hkv) * D;
  const int half = D / 2;
  const int64_t capacity = kv.max_blocks * kv.block_size;

  // Epilogue operands do not depend on the GEMM: fetch them first (position, then the rotary
  // coefficients, the bias pair and the cache block of this thread's (pair, row) items).
  constexpr int kPairs = (Core::kTileN / 2) * Core::kTileM;
  constexpr int kItems = (kPairs + kNormThreads - 1) / kNormThreads;
  int64_t pos[kItems];
  float cs[kItems][2], bs[kItems][2];
  int64_t blk[kItems];
#pragma unroll
  for (int it = 0; it < kItems; ++it) {
    const int idx = threadIdx.x + it * kNormThreads;
    const int m = idx % Core::kTileM;
    pos[it] = (idx < kPairs && m < M) ? loadIndex(positions, pos64, m) : -1;
  }
#pragma unroll
  for (int it = 0; it < kItems; ++it) {
    const int idx = threadIdx.x + it * kNormThreads;
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

  tileLoop<1, MB, kNormWaves, kNormUnroll>(w, XGlobal{x, K}, N, K, M, lds, norm_w, eps, [&](int64_t) {
#pragma unroll
  for (int it = 0; it < kItems; ++it) {
    const int idx = threadIdx.x + it * kNormThreads;
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
  });
}

// out = residual + bf16(x W^T + b); 16 weight rows per workgroup, 8 waves split K.
template <int MB>
__device__ void linear_residual_impl(const uint16_t* x, const uint16_t* w, const uint16_t* bias,
                                     const uint16_t* residual, uint16_t* out, int M, int64_t N,
                                     int K) {
  using Core = SkinnyCore<1, MB, kResWaves, (MB >= 4 ? 2 : 4)>;  // 256 VGPRs at 512 threads
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
  Core::run(w, XGlobal{x, K}, N, K, M, n0, 0, K / 64, lds);
#pragma unroll
  for (int it = 0; it < kItems; ++it) {
    const int idx = threadIdx.x + it * kThreadsRes;
    const int nl = idx / Core::kTileM, m = idx % Core::kTileM;
    const int64_t n = n0 + nl;
    if (idx >= Core::kTileN * Core::kTileM || m >= M || n >= N) continue;
    float y = lds[idx];
    if (bias != nullptr) y += bf16ToFloat(bias[n]);
    out[m * N + n] = floatToBf16(res[it] + roundBf16(y));
  }
}

// out = residual + bf16(x W^T + b) with K split over grid.y (16 weight rows per workgroup):
// every split stores its partial tile with agent-scope stores and arrives at counters[tile];
// the last split to arrive sums the partials in split order, writes the output tile and resets
// the counter to zero. No cross-workgroup fence and no second kernel. splits <= kMaxNormSplits.
//   partials: [tiles][splits][16 x 16 MB] fp32, counters: [tiles] (zero before the first call)
template <int MB>
__device__ void linear_residual_splitk_impl(const uint16_t* x, const uint16_t* w,
                                            const uint16_t* bias, const uint16_t* residual,
                                            uint16_t* out, int M, int64_t N, int K, int splits,
                                            float* partials, unsigned* counters) {
  using Core = SkinnyCore<1, MB, kWaves>;
  constexpr int kElems = Core::kTileN * Core::kTileM;
  constexpr int kItems = (kElems + kThreads - 1) / kThreads;
  __shared__ float lds[Core::kLdsFloats];
  __shared__ int is_last;
  const int64_t n0 = static_cast<int64_t>(blockIdx.x) * Core::kTileN;
  float res[kItems], bv[kItems];
#pragma unroll
  for (int it = 0; it < kItems; ++it) {  // residual and bias fetched before the weights
    const int idx = threadIdx.x + it * kThreads;
    const int nl = idx / Core::kTileM, m = idx % Core::kTileM;
    const int64_t n = n0 + nl;
    const bool live = idx < kElems && m < M && n < N;
    res[it] = live ? bf16ToFloat(residual[m * N + n]) : 0.f;
    bv[it] = live && bias != nullptr ? bf16ToFloat(bias[n]) : 0.f;
  }
  int sb, se;
  splitRange(K / 64, blockIdx.y, splits, sb, se);
  Core::run(w, XGlobal{x, K}, N, K, M, n0, sb, se, lds);
  float* base = partials + static_cast<int64_t>(blockIdx.x) * splits * kElems;
  for (int idx = threadIdx.x; idx < kElems; idx += blockDim.x)
    __hip_atomic_store(base + static_cast<int64_t>(blockIdx.y) * kElems + idx, lds[idx],
                       __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
  // Arrive: every partial store of this workgroup has completed before the counter moves.
  asm volatile("s_waitcnt vmcnt(0)" ::: "memory");
  __syncthreads();
  if (threadIdx.x == 0) {
    const unsigned old = __hip_atomic_fetch_add(counters + blockIdx.x, 1u, __ATOMIC_RELAXED,
                                                __HIP_MEMORY_SCOPE_AGENT);
    is_last = old + 1 == static_cast<unsigned>(splits);
    if (is_last)
      __hip_atomic_store(counters + blockIdx.x, 0u, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
  }
  __syncthreads();
  if (!is_last) return;
#pragma unroll
  for (int it = 0; it < kItems; ++it) {
    const int idx = threadIdx.x + it * kThreads;
    if (idx >= kElems) continue;
    float part[kMaxNormSplits];
#pragma unroll
    for (int sp = 0; sp < kMaxNormSplits; ++sp)  // all loads first: their round trips overlap
      part[sp] = sp < splits ? __hip_atomic_load(base + sp * kElems + idx, __ATOMIC_RELAXED,
                                                 __HIP_MEMORY_SCOPE_AGENT)
                             : 0.f;
    const int nl = idx / Core::kTileM, m = idx % Core::kTileM;
    const int64_t n = n0 + nl;
    if (m >= M || n >= N) continue;
    float y = part[0];
#pragma unroll
    for (int sp = 1; sp < kMaxNormSplits; ++sp) y += part[sp];  // split order; absent = +0
    out[m * N + n] = floatToBf16(res[it] + roundBf16(y + bv[it]));
  }
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
  for (int idx = threadIdx.x; idx < Core::kTileN * Core::kTileM; idx += blockDim.x) {
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
  __shared__ float lds[Core::kLdsFloats];
  tileLoop<2, MB, kNormWaves, kNormUnroll>(w_gu, XGlobal{x, K}, 2 * F, K, M, lds, norm_w, eps,
                                           [&](int64_t t) {
    const int64_t f0 = t * 16;  // tile t = gate rows [16t, 16t+16) then up rows [16t, 16t+16)
    for (int idx = threadIdx.x; idx < 16 * Core::kTileM; idx += blockDim.x) {
      const int j = idx % 16, m = idx / 16;
      const int64_t f = f0 + j;
      if (m >= M || f >= F) continue;
      const float g = roundBf16(lds[j * Core::kTileM + m]);
      const float u = roundBf16(lds[(16 + j) * Core::kTileM + m]);
      const float s = roundBf16(g / (1.0f + expf(-g)));
      out[m * F + f] = floatToBf16(s * u);
    }
  });
}

constexpr int kLmTileN = 32;  // vocab rows per lm_head tile (NF = 2)
constexpr int kLmQuarters = kLmTileN / 4;

// Logits of vocab tiles of 32 rows (grid-strided over the workgroups) plus each tile's argmax
// partial per row: part_*[m * tiles + t]. Requires K / 64 <= 4 * kWaves.
template <int MB>
__device__ void lm_head_argmax_impl(const uint16_t* xn, const uint16_t* w, void* logits,
                                    int logits_f32, float* part_val, int32_t* part_idx, int M,
                                    int64_t V, int K) {
  using Core = SkinnyCore<2, MB, kWaves>;
  static_assert(Core::kTileN == kLmTileN, "lm_head tile");
  __shared__ float lds[Core::kLdsFloats + kLmQuarters * Core::kTileM];
  __shared__ int lds_arg[kLmQuarters * Core::kTileM];
  const int64_t tiles = (V + Core::kTileN - 1) / Core::kTileN;
  tileLoop<2, MB, kWaves, 4>(w, XGlobal{xn, K}, V, K, M, lds, nullptr, 0.f, [&](int64_t t) {
    const int64_t n0 = t * Core::kTileN;
    if (logits != nullptr) {
      for (int idx = threadIdx.x; idx < Core::kTileN * Core::kTileM; idx += blockDim.x) {
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
    for (int idx = threadIdx.x; idx < kLmQuarters * Core::kTileM; idx += blockDim.x) {
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
    for (int m = threadIdx.x; m < M; m += blockDim.x) {
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
  for (int t0 = threadIdx.x; t0 < tiles; t0 += kBatch * blockDim.x) {
    float v[kBatch];
    int32_t ix[kBatch];
#pragma unroll
    for (int u = 0; u < kBatch; ++u) {
      const int t = t0 + u * blockDim.x;
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
    qkv_rope_append_impl<MB>(x, norm_w, eps, w, bias, cos_t, sin_t, max_pos, positions, pos64,    \
                             q_out, KvCacheArgs{k_pool, v_pool, block_table, block_size,          \
                                                max_blocks},                                      \
                             M, K, Hq, Hkv, D);                                                   \
  }                                                                                               \
  extern "C" __global__ void __launch_bounds__(kResWaves * 64) linear_residual_m##MB(             \
      const uint16_t* x, const uint16_t* w, const uint16_t* bias, const uint16_t* residual,       \
      uint16_t* out, int M, int64_t N, int K) {                                                   \
    linear_residual_impl<MB>(x, w, bias, residual, out, M, N, K);                                 \
  }                                                                                               \
  extern "C" __global__ void __launch_bounds__(kThreads) linear_residual_splitk_m##MB(            \
      const uint16_t* x, const uint16_t* w, const uint16_t* bias, const uint16_t* residual,       \
      uint16_t* out, int M, int64_t N, int K, int splits, float* partials, unsigned* counters) {  \
    linear_residual_splitk_impl<MB>(x, w, bias, residual, out, M, N, K, splits, partials,         \
                                    counters);                                                    \
  }                                                                                               \
  extern "C" __global__ void __launch_bounds__(kThreads) linear_partial_m##MB(                    \
      const uint16_t* x, const uint16_t* w, float* partials, int M, int64_t N, int K,             \
      int splits) {                                                                               \
    linear_partial_impl<MB>(x, w, partials, M, N, K, splits);                                     \
  }                                                                                               \
  extern "C" __global__ void __launch_bounds__(kNormThreads) gate_up_silu_m##MB(                  \
      const uint16_t* x, const uint16_t* norm_w, float eps, const uint16_t* w_gu, uint16_t* out,  \
      int M, int64_t F, int K) {                                                                  \
    gate_up_silu_impl<MB>(x, norm_w, eps, w_gu, out, M, F, K);                                    \
  }                                                                                               \
  extern "C" __global__ void __launch_bounds__(kThreads) lm_head_argmax_m##MB(                    \
      const uint16_t* xn, const uint16_t* w, void* logits, int logits_f32, float* part_val,       \
      int32_t* part_idx, int M, int64_t V, int K) {                                               \
    lm_head_argmax_impl<MB>(xn, w, logits, logits_f32, part_val, part_idx, M, V, K);              \
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
