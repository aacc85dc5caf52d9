#pragma once

// Stage building blocks of a Qwen2-style decoder layer in bf16, shared by the one-stage kernels
// (decode.hip) and the persistent decoder-stack kernel (stack.hip), so that both compute every
// tile with the same instructions in the same order and give bit-identical results:
//
//   normalizeFragments  RMSNorm of x fragments held in registers (rms_norm/kernel.py:6-14)
//   tileLoop            grid-strided weight tiles against one x kept in registers
//   QkvEpilogue         bias, interleaved RoPE (rotary/kernel.py:6-35), q out, k/v into the
//                       paged KV cache at each row's position
//   gateUpEpilogue      bf16(bf16(silu(gate)) * up) of one 16-output block
//   ResidualTile        out = residual + bf16(y + b) of one 16-row tile
//   splitKArrive        split-K partial tile store + last-arriver merge into out
//
// Every node of the unfused graph rounds its output to bf16; these helpers keep those rounding
// points. Mem (skinny.h) selects plain or agent-scope accesses for data another workgroup of
// the same launch produces or consumes.
#include "common.h"
#include "skinny.h"

namespace dk {

// RMSNorm-prologue GEMMs (qkv, gate_up): 8 waves, two per SIMD, so one wave's normalize VALU
// runs while the other is held issuing its weight loads; 8 waves x 2 steps x 64 columns covers
// hidden <= 1024.
constexpr int kNormWaves = 8;
constexpr int kNormThreads = kNormWaves * kWave;
constexpr int kNormUnroll = 2;
// linear_residual (o_proj, down_proj): 8 waves split K inside a workgroup.
constexpr int kResWaves = 8;
constexpr int kResThreads = kResWaves * kWave;
constexpr int kMaxSplits = 8;  // split-K partials summed by the last arriver
// Split-K linear_residual (down_proj): waves without K steps. The decoder stack's down_proj
// units poll the gate_up counter from wave 0, whose poll then does not queue behind weight
// loads; the one-stage kernel uses the same split of K over waves, so both sum alike.
constexpr int kDownIdle = 1;

__device__ __forceinline__ float roundBf16(float v) { return bf16ToFloat(floatToBf16(v)); }

// Steps [begin, end) of split `split` out of `splits` over `steps` 64-column steps.
__device__ __forceinline__ void splitRange(int steps, int split, int splits, int& begin, int& end) {
  const int per = (steps + splits - 1) / splits;
  begin = split * per;
  end = begin + per < steps ? begin + per : steps;
}

struct KvCacheArgs {
  uint16_t* k_pool;
  uint16_t* v_pool;
  const int32_t* block_table;
  int64_t block_size;
  int64_t max_blocks;
};

// RMSNorm weights of the 64-column steps a wave holds (see normalizeFragments), requested
// ahead of x: they do not depend on it.
template <int kW, int kU>
__device__ __forceinline__ void loadNormWeights(U128 (&wv)[kU][2], const uint16_t* norm_w,
                                                int wave, int steps, int g) {
#pragma unroll
  for (int u = 0; u < kU; ++u) {
    const int s = wave + u * kW;
    if (s >= steps) break;  // uniform: wave comes from readfirstlane
    const int64_t k0 = static_cast<int64_t>(s) * 64 + g * 8;
    wv[u][0] = gload16(norm_w + k0);
    wv[u][1] = gload16(norm_w + k0 + 32);
  }
}

// LDS floats of the RMSNorm row-sum exchange (kept apart from the tile reductions' LDS).
template <int MB, int kW>
constexpr int kNormLdsFloats = kW * 16 * MB;

// RMSNorm of x fragments held in registers, every 64-column step of K being in `xb` (lanes of
// wave w hold steps w, w + kW, ...), with the norm weights wv (loadNormWeights):
// x[m, k] <- bf16(x[m, k] * rsqrt(mean_k x[m, k]^2 + eps) * w[k]) (rms_norm/kernel.py:6-14).
// Row sums of squares are reduced over the 4 lanes of a row and then over the waves through
// norm_lds (kNormLdsFloats<MB, kW> floats, not touched by anything else in between) in a fixed
// order.
template <int NF, int MB, int kW, int kU>
__device__ __forceinline__ void normalizeFragments(
    typename SkinnyCore<NF, MB, kW, kU>::XBatch& xb, const U128 (&wv)[kU][2], int K, float eps,
    float* norm_lds, int wave, int steps, int r, int g) {
  FP_EXACT;
  float sq[MB];
#pragma unroll
  for (int b = 0; b < MB; ++b) {
    sq[b] = 0.f;
#pragma unroll
    for (int u = 0; u < kU; ++u) {
      if (wave + u * kW >= steps) break;
#pragma unroll
      for (int h = 0; h < 2; ++h) {
        // x0^2 + x1^2 + sq in one instruction (v_dot2c_f32_bf16; bf16 squares are exact). The
        // pairs are taken from the whole fragment viewed as 8 bf16: bit-casting one 32-bit
        // element of the fragment to bf16x2 instead is mis-folded by this compiler (every
        // element reads element 0).
        const bf16x8 all = __builtin_bit_cast(bf16x8, xb.x[u][b][h]);
#pragma unroll
        for (int e = 0; e < 4; ++e) {
          const bf16x2_t v = {all[2 * e], all[2 * e + 1]};
          sq[b] = __builtin_amdgcn_fdot2_f32_bf16(v, v, sq[b], false);
        }
      }
    }
    sq[b] = rowsSum(sq[b]);
    if (g == 0) norm_lds[wave * 16 * MB + b * 16 + r] = sq[b];
  }
  __syncthreads();
  float inv[MB];
#pragma unroll
  for (int b = 0; b < MB; ++b) {
    float total = 0.f;
#pragma unroll
    for (int v = 0; v < kW; ++v) total += norm_lds[v * 16 * MB + b * 16 + r];
    inv[b] = 1.0f / sqrtf(total / static_cast<float>(K) + eps);
  }
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

// Weight tiles t = t_first, t_first + t_stride, ... below t_end (16 * NF rows each) against one x whose
// fragments are loaded once (and RMS-normalized with norm_w when it is non-NULL) and stay in
// registers; the next tile's weights stream in while the current one is multiplied. epi(t)
// reads the reduced tile [16 NF][16 MB] from lds (row n, column m at lds[n * 16 MB + m]).
// lds holds Core::kLdsFloats floats, plus kNormLdsFloats<MB, kW> after them when norm_w is
// non-NULL. Requires K / 64 <= kU * kW.
//
// Load order. With an ungated x (kGated false) x and the norm weights are requested first:
// loads complete in issue order, so the RMSNorm of x (VALU) overlaps the weight stream instead
// of waiting behind it. With kGated the first two tiles' weights and the norm weights are
// requested, then gate() waits until another workgroup has produced x, and x is loaded with
// Mem. The arithmetic is the same either way.
//
// mark(p) (every thread calls it) marks points for a timeline: 2 once x is requested, 0 once x
// is loaded (and normalized), 1 when the first tile is reduced. xs: XGlobal (row-major) or XFrag
// (fragment order).
template <int NF, int MB, int kW, int kU, class Mem = PlainMem, bool kGated = false,
          bool kLazySum = false, class Gate = NoWait, typename Epi, class Mark = NoMark,
          class XS = XGlobal>
__device__ __forceinline__ void tileLoop(const uint16_t* w, const XS& xs, int64_t N, int K,
                                         int M, float* lds, const uint16_t* norm_w, float eps,
                                         int64_t t_first, int64_t t_stride, int64_t t_end,
                                         Gate&& gate, Epi&& epi, Mark mark = Mark{}) {
  using Core = SkinnyCore<NF, MB, kW, kU>;
  const int lane = freshThreadIdx() % kWave;
  const int wave = __builtin_amdgcn_readfirstlane(threadIdx.x / kWave);
  const int r = lane % 16, g = lane / 16;
  const int steps = K / 64;
  const int64_t all_tiles = (N + Core::kTileN - 1) / Core::kTileN;
  const int64_t tiles = t_end < all_tiles ? t_end : all_tiles;
  const int64_t stride = t_stride;
  int64_t t = t_first;
  if (t >= tiles) return;
  typename Core::WBatch bufA, bufB;
  typename Core::XBatch xb;
  U128 wv[kU][2];
  if (!kGated) {
    Core::template issueX<Mem>(xb, Core::xrows(xs, M, r, g), wave, steps);
    if (norm_w != nullptr) loadNormWeights<kW, kU>(wv, norm_w, wave, steps, g);
  }
  Core::issueW(bufA, Core::rows(w, N, K, t * Core::kTileN, r, g), wave, steps);
  if (t + stride < tiles)
    Core::issueW(bufB, Core::rows(w, N, K, (t + stride) * Core::kTileN, r, g), wave, steps);
  if (kGated) {
    if (norm_w != nullptr) loadNormWeights<kW, kU>(wv, norm_w, wave, steps, g);
    gate();
    Core::template issueX<Mem>(xb, Core::xrows(xs, M, r, g), wave, steps);
  }
  float* const norm_lds = lds + Core::kLdsFloats;
  mark(2);  // x issued (a tracing caller may wait for it here)
  if (norm_w != nullptr)
    normalizeFragments<NF, MB, kW, kU>(xb, wv, K, eps, norm_lds, wave, steps, r, g);
  mark(0);
  auto tile = [&](const typename Core::WBatch& wb, int64_t tt) {
    f32x4 acc[NF][MB];
    Core::zero(acc);
    Core::compute(acc, wb, xb, wave, steps);
    if constexpr (kLazySum)
      Core::storePartials(acc, lds, r, g, wave);  // epi adds the wave slices (partialSum)
    else
      Core::reduce(acc, lds, r, g, wave);
    if (tt == t_first) mark(1);
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

// ---- qkv: bias, RoPE, q out, k/v into the paged cache -------------------------------------

struct QkvParams {
  const uint16_t* bias;  // [(Hq + 2 Hkv) D] or NULL
  const float* cos_t;    // [max_pos, D / 2]
  const float* sin_t;
  int64_t max_pos;
  const void* positions;  // [M] int32/int64: the slot each row's new token is written to
  int pos64;
  uint16_t* q_out;  // [M, Hq, D]
  KvCacheArgs kv;
  int M, Hq, Hkv, D;
  // When set, q goes here instead of q_out: [M, Hq, D / 2] tagged words (storeTaggedBits), each
  // the bf16 pair (d, d + 1) with tag q_tag, for a reader that polls the words themselves.
  uint64_t* q_tagged = nullptr;
  unsigned q_tag = 0;
};

enum : int { kQkvAll = 0, kQkvQ = 1, kQkvCache = 2 };

// Operands of one QkvEpilogue thread item, parked in LDS (QkvEpilogue<..., true>).
struct QkvParked {
  int64_t pos;
  float c, s, b0, b1;
  int32_t blk;  // a block_table entry, or -1
  int32_t unused;
};

// Epilogue of one 16-row tile of the [q | k | v] projection (kNormThreads threads). Thread item
// (pair, m) owns output columns n0 + 2 pair, n0 + 2 pair + 1 of row m: a RoPE pair
// (rotary/kernel.py:6-35 rotates interleaved pairs). The operands that do not depend on the GEMM
// (position, rotary coefficients, bias, cache block) are fetched by prefetch() before it.
// kParked: prefetch() waits for them and parks them in LDS at park[0, kPairs) (each thread its
// own slots, so no barrier), instead of holding them in registers across the tile's GEMM, where
// a kernel short of registers spills them and reloads each from scratch with a full wait.
template <int MB, class Mem, bool kParked = false>
struct QkvEpilogue {
  static constexpr int kTileN = 16;
  static constexpr int kTileM = 16 * MB;
  static constexpr int kPairs = (kTileN / 2) * kTileM;
  static constexpr int kItems = (kPairs + kNormThreads - 1) / kNormThreads;
  int64_t pos[kItems];
  float cs[kItems][2], bs[kItems][2];
  int64_t blk[kItems];
  QkvParked* park = nullptr;  // kParked: kPairs slots

  __device__ __forceinline__ void prefetch(const QkvParams& p, int64_t n0) {
    FP_EXACT;
    const int64_t N = static_cast<int64_t>(p.Hq + 2 * p.Hkv) * p.D;
    const int64_t q_rows = static_cast<int64_t>(p.Hq) * p.D;
    const int64_t k_rows = static_cast<int64_t>(p.Hkv) * p.D;
    const int half = p.D / 2;
    const int64_t capacity = p.kv.max_blocks * p.kv.block_size;
#pragma unroll
    for (int it = 0; it < kItems; ++it) {
      const int idx = freshThreadIdx() + it * kNormThreads;
      const int m = idx % kTileM;
      pos[it] = (idx < kPairs && m < p.M) ? loadIndex(p.positions, p.pos64, m) : -1;
    }
#pragma unroll
    for (int it = 0; it < kItems; ++it) {
      const int idx = freshThreadIdx() + it * kNormThreads;
      const int pair = idx / kTileM, m = idx % kTileM;
      const int64_t n = n0 + 2 * pair;
      const bool live = pos[it] >= 0 && n < N;
      // column within the q, k or v block: below (Hq + 2 Hkv) D, so 32-bit arithmetic is exact
      const int local = static_cast<int>(
          n < q_rows ? n : (n < q_rows + k_rows ? n - q_rows : n - q_rows - k_rows));
      const int d = local % p.D;
      const bool rot = live && n < q_rows + k_rows && pos[it] < p.max_pos;
      cs[it][0] = rot ? gp(p.cos_t)[pos[it] * half + d / 2] : 1.f;
      cs[it][1] = rot ? gp(p.sin_t)[pos[it] * half + d / 2] : 0.f;
      bs[it][0] = (live && p.bias != nullptr) ? bf16ToFloat(gp(p.bias)[n]) : 0.f;
      bs[it][1] = (live && p.bias != nullptr) ? bf16ToFloat(gp(p.bias)[n + 1]) : 0.f;
      blk[it] = (live && n >= q_rows && pos[it] < capacity)
                    ? gp(p.kv.block_table)[m * p.kv.max_blocks + pos[it] / p.kv.block_size]
                    : -1;
      if constexpr (kParked) {
        if (idx < kPairs)
          park[idx] = QkvParked{pos[it],   cs[it][0], cs[it][1], bs[it][0],
                                bs[it][1], static_cast<int32_t>(blk[it]), 0};
      }
    }
  }

  // kOutputs selects what is written: kQkvAll, kQkvQ (q only) or kQkvCache (k/v into the cache
  // only); values are computed identically in every case.
  template <int kOutputs = 0>
  __device__ __forceinline__ void apply(const QkvParams& p, int64_t n0, const float* lds) const {
    FP_EXACT;
    const int64_t N = static_cast<int64_t>(p.Hq + 2 * p.Hkv) * p.D;
    const int64_t q_rows = static_cast<int64_t>(p.Hq) * p.D;
    const int64_t k_rows = static_cast<int64_t>(p.Hkv) * p.D;
#pragma unroll
    for (int it = 0; it < kItems; ++it) {
      const int idx = freshThreadIdx() + it * kNormThreads;
      const int pair = idx / kTileM;
      const int m = idx % kTileM;
      const int64_t n = n0 + 2 * pair;
      QkvParked o;
      if constexpr (kParked) {
        if (idx >= kPairs) continue;
        o = park[idx];
      } else {
        o = QkvParked{pos[it], cs[it][0], cs[it][1], bs[it][0], bs[it][1], 0, 0};
      }
      const int64_t blk_it = kParked ? static_cast<int64_t>(o.blk) : blk[it];
      if (o.pos < 0 || n >= N) continue;
      // linear output (bias added, rounded), then the rotation in fp32, rounded again
      float v0 = roundBf16(lds[(2 * pair) * kTileM + m] + o.b0);
      float v1 = roundBf16(lds[(2 * pair + 1) * kTileM + m] + o.b1);
      const bool is_q = n < q_rows;
      const bool is_k = !is_q && n < q_rows + k_rows;
      if ((kOutputs == kQkvQ && !is_q) || (kOutputs == kQkvCache && is_q)) continue;
      const int local = static_cast<int>(is_q ? n : (is_k ? n - q_rows : n - q_rows - k_rows));
      const int head = local / p.D;
      const int d = local % p.D;
      if (is_q || is_k) {
        const float r0 = v0 * o.c - v1 * o.s;
        const float r1 = v0 * o.s + v1 * o.c;
        v0 = r0;
        v1 = r1;
      }
      const uint32_t packed = packBf16x2(v0, v1);
      if (is_q) {
        const int64_t at = (static_cast<int64_t>(m) * p.Hq + head) * p.D + d;
        if (p.q_tagged != nullptr)
          storeTaggedBits(p.q_tagged + at / 2, packed, p.q_tag);
        else
          Mem::storeU32(reinterpret_cast<uint32_t*>(p.q_out + at), packed);
        continue;
      }
      if (blk_it < 0) continue;
      const int64_t off = o.pos % p.kv.block_size;
      if (is_k) {
        uint16_t* dst =
            p.kv.k_pool + ((blk_it * p.Hkv + head) * p.kv.block_size + off) * p.D + d;
        Mem::storeU32(reinterpret_cast<uint32_t*>(dst), packed);
      } else {
        uint16_t* dst =
            p.kv.v_pool + ((blk_it * p.Hkv + head) * p.D + d) * p.kv.block_size + off;
        Mem::storeU16(dst, static_cast<uint16_t>(packed));
        Mem::storeU16(dst + p.kv.block_size, static_cast<uint16_t>(packed >> 16));
      }
    }
  }
};

// ---- gate_up: SwiGLU of one 16-output block ----------------------------------------------

// Tile t of the interleaved gate/up weight = gate rows [16t, 16t+16) then up rows [16t, 16t+16);
// lds holds the reduced [32][16 MB] tile, or with kLazySum the waves' partial tiles, which are
// added here (SkinnyCore::partialSum: the sum reduce() forms, in its order).
// out[m, f] = bf16(bf16(silu(bf16 gate)) * bf16 up).
// frag_steps > 0: out is in fragment order (fragOffset) with F / 64 steps.
template <int MB, class Mem, bool kLazySum = false>
__device__ __forceinline__ void gateUpEpilogue(const float* lds, uint16_t* out, int M, int64_t F,
                                               int64_t t, int frag_steps = 0) {
  FP_EXACT;
  using Core = SkinnyCore<2, MB, kNormWaves, kNormUnroll>;
  constexpr int kTileM = 16 * MB;
  const int64_t f0 = t * 16;
  auto at = [&](int n, int m) { return kLazySum ? Core::partialSum(lds, n, m) : lds[n * kTileM + m]; };
  for (int idx = freshThreadIdx(); idx < 16 * kTileM; idx += kNormThreads) {
    const int j = idx % 16, m = idx / 16;
    const int64_t f = f0 + j;
    if (m >= M || f >= F) continue;
    const float g = roundBf16(at(j, m));
    const float u = roundBf16(at(16 + j, m));
    const float s = roundBf16(g / (1.0f + expf(-g)));
    Mem::storeU16(out + actOffset(m, f, F, frag_steps), floatToBf16(s * u));
  }
}

// ---- residual update of one 16-row tile ---------------------------------------------------

// out[m, n] = bf16(residual[m, n] + bf16(y[n][m] + b[n])) for the tile at weight row n0, with
// kThreadsT threads; load() fetches the residual (and bias) so they can be requested early.
// Thread item (m, half) owns the 8 consecutive outputs n0 + 8 half, ..., + 7 of row m, so a row
// segment is read and written with one 16-byte access when N is a multiple of 8 and the
// pointers are 16-byte aligned (element by element otherwise); the values are the same either
// way. frag_steps > 0: residual / out are in fragment order (fragOffset, N / 64 steps), where a
// row segment of 8 outputs is contiguous too.
template <int MB, int kThreadsT, class Mem>
struct ResidualTile {
  static constexpr int kTileN = 16;
  static constexpr int kTileM = 16 * MB;
  static constexpr int kElems = kTileN * kTileM;
  static constexpr int kItems = 2 * kTileM;
  static_assert(kItems <= kThreadsT, "one item per thread");
  float res[8], bv[8];

  __device__ __forceinline__ static bool vectorOk(const void* p, int64_t N) {
    return N % 8 == 0 && (reinterpret_cast<uintptr_t>(p) & 15u) == 0;
  }

  __device__ __forceinline__ void load(const uint16_t* residual, const uint16_t* bias, int64_t n0,
                                       int M, int64_t N, int frag_steps = 0) {
    const int idx = freshThreadIdx();
    const int m = idx / 2;
    const int64_t n = n0 + 8 * (idx % 2);
    const bool live = idx < kItems && m < M;
    if (live && n + 8 <= N && vectorOk(residual, N)) {
      const U128 r = Mem::load16(residual + actOffset(m, n, N, frag_steps));
#pragma unroll
      for (int e = 0; e < 4; ++e) {
        res[2 * e] = bf16ToFloat(static_cast<uint16_t>(r[e]));
        res[2 * e + 1] = bf16ToFloat(static_cast<uint16_t>(r[e] >> 16));
      }
    } else {
#pragma unroll
      for (int j = 0; j < 8; ++j)
        res[j] = live && n + j < N
                     ? bf16ToFloat(Mem::loadU16(residual + actOffset(m, n + j, N, frag_steps)))
                     : 0.f;
    }
#pragma unroll
    for (int j = 0; j < 8; ++j)
      bv[j] = live && bias != nullptr && n + j < N ? bf16ToFloat(gp(bias)[n + j]) : 0.f;
  }

  // y(e) returns the fp32 GEMM result of tile element e = nl * kTileM + m (row nl, column m).
  template <class Y>
  __device__ __forceinline__ void store(uint16_t* out, int64_t n0, int M, int64_t N, Y&& y,
                                        int frag_steps = 0) const {
    FP_EXACT;
    const int idx = freshThreadIdx();
    const int m = idx / 2, half = idx % 2;
    const int64_t n = n0 + 8 * half;
    if (idx >= kItems || m >= M) return;
    float v[8];
#pragma unroll
    for (int j = 0; j < 8; ++j) v[j] = res[j] + roundBf16(y((8 * half + j) * kTileM + m) + bv[j]);
    if (n + 8 <= N && vectorOk(out, N)) {
      U128 o;
#pragma unroll
      for (int e = 0; e < 4; ++e) o[e] = packBf16x2(v[2 * e], v[2 * e + 1]);
      Mem::store16(out + actOffset(m, n, N, frag_steps), o);
      return;
    }
#pragma unroll
    for (int j = 0; j < 8; ++j)
      if (n + j < N) Mem::storeU16(out + actOffset(m, n + j, N, frag_steps), floatToBf16(v[j]));
  }
};

// Split-K tail of one 16-row tile whose reduced partial is in lds: the partial is stored with
// agent-scope stores to partials[split] (layout [splits][16 x 16 MB]) and the workgroup arrives
// at *counter. The workgroup that brings the counter to `arrivals` is the last one: it reads
// every split's partial with agent-scope loads (all issued before any is used), sums them in
// split order, writes out = residual + bf16(sum + b) through rt, resets the counter to zero when
// `reset` is set, and returns true. No cross-workgroup fence is needed: agent-scope stores and
// loads bypass the non-coherent L2, and s_waitcnt vmcnt(0) orders the partial stores before the
// counter update.
template <int MB, int kThreadsT, class Mem>
__device__ __forceinline__ bool splitKArrive(const float* lds, float* partials, int split,
                                             int splits, unsigned* counter, unsigned arrivals,
                                             bool reset, const ResidualTile<MB, kThreadsT, Mem>& rt,
                                             uint16_t* out, int64_t n0, int M, int64_t N,
                                             int* is_last) {
  FP_EXACT;
  constexpr int kElems = 16 * 16 * MB;
  for (int idx = freshThreadIdx(); idx < kElems; idx += kThreadsT)
    __hip_atomic_store(gp(partials) + static_cast<int64_t>(split) * kElems + idx, lds[idx],
                       __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
  asm volatile("s_waitcnt vmcnt(0)" ::: "memory");
  __syncthreads();
  if (threadIdx.x == 0) {
    const unsigned old =
        __hip_atomic_fetch_add(gp(counter), 1u, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
    *is_last = old + 1 == arrivals;
    if (*is_last && reset)
      __hip_atomic_store(gp(counter), 0u, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
  }
  __syncthreads();
  if (!*is_last) return false;
  // The sums replace this workgroup's own partial in lds (every thread has stored it above).
  float* const sums = const_cast<float*>(lds);
  for (int idx = freshThreadIdx(); idx < kElems; idx += kThreadsT) {
    float part[kMaxSplits];
#pragma unroll
    for (int sp = 0; sp < kMaxSplits; ++sp)
      part[sp] = sp < splits ? __hip_atomic_load(gp(partials) + sp * kElems + idx, __ATOMIC_RELAXED,
                                                 __HIP_MEMORY_SCOPE_AGENT)
                             : 0.f;
    float y = part[0];
#pragma unroll
    for (int sp = 1; sp < kMaxSplits; ++sp) y += part[sp];  // split order; absent = +0
    sums[idx] = y;
  }
  __syncthreads();
  rt.store(out, n0, M, N, [&](int e) { return sums[e]; });
  return true;
}

// Split-K tail for a persistent launch (every workgroup resident at once), no counter: split
// s > 0 stores its reduced partial (lds) as tagged words (storeTagged) and returns false; split 0
// adds the other splits' words to its own partial in split order as they arrive (loadTagged),
// writes out = residual + bf16(sum + b) through rt and returns true. The sums are those of
// splitKArrive, bit for bit. partials: this tile's [splits][16 x 16 MB] tagged words.
// out_frag_steps: out's layout (ResidualTile::store).
template <int MB, int kThreadsT, class Mem>
__device__ __forceinline__ bool splitKTagged(float* lds, uint64_t* partials, int split,
                                             int splits, unsigned tag, unsigned* abort_word,
                                             const ResidualTile<MB, kThreadsT, Mem>& rt,
                                             uint16_t* out, int64_t n0, int M, int64_t N,
                                             int out_frag_steps = 0) {
  FP_EXACT;
  constexpr int kElems = 16 * 16 * MB;
  if (split != 0) {
    for (int idx = freshThreadIdx(); idx < kElems; idx += kThreadsT)
      storeTagged(partials + static_cast<int64_t>(split) * kElems + idx, lds[idx], tag);
    return false;
  }
  for (int idx = freshThreadIdx(); idx < kElems; idx += kThreadsT) {
    const uint64_t* ptr[kMaxSplits - 1];
#pragma unroll
    for (int sp = 1; sp < kMaxSplits; ++sp)
      ptr[sp - 1] = partials + static_cast<int64_t>(sp < splits ? sp : 0) * kElems + idx;
    float part[kMaxSplits - 1];
    loadTagged<kMaxSplits - 1>(part, ptr, splits - 1, tag, abort_word);
    float y = lds[idx];
#pragma unroll
    for (int sp = 1; sp < kMaxSplits; ++sp) y += sp < splits ? part[sp - 1] : 0.f;  // split order
    lds[idx] = y;
  }
  __syncthreads();
  rt.store(out, n0, M, N, [&](int e) { return lds[e]; }, out_frag_steps);
  return true;
}

}  // namespace dk
