#pragma once

// Weight-streaming MFMA core for skinny GEMMs on gfx950: out[m, n] = sum_k x[m, k] * w[n, k]
// with few rows m (decode batch, M <= 16 * MB) and a large bf16 weight w [N, K] read once.
//
// Work split
//   - A workgroup owns an N-tile of 16 * NF weight rows and a slice of K (grid.y splits K).
//   - Its kWaves waves split that slice further, each walking 64-column steps: per step a lane
//     loads two 16-byte runs of one weight row, so every wave-wide load pair covers 16 rows x
//     128 contiguous bytes (whole cache lines, each byte fetched once).
//   - x fragments come from global memory (x is small and stays in L2) or from an LDS copy
//     (used when a prologue has produced x inside the workgroup, e.g. RMSNorm).
//   - MFMA v_mfma_f32_16x16x32_bf16: A = 16 weight rows x 32 k, B = 32 k x 16 batch rows.
//     Lane l holds A[l % 16][(l / 16) * 8 + j] and B[(l / 16) * 8 + j][l % 16], j < 8, and
//     receives D[(l / 16) * 4 + i][l % 16], i < 4. A and B use the same k order, so the
//     assignment of k to lanes only has to agree between the two operands.
//   - Partial tiles of the waves are summed in LDS in a fixed order, so results do not depend
//     on timing. The reduced fp32 tile [16 * NF][16 * MB] is left in LDS for an epilogue.

#include "common.h"

namespace dk {

typedef __bf16 bf16x8 __attribute__((ext_vector_type(8)));
typedef float f32x4 __attribute__((ext_vector_type(4)));

struct alignas(16) U128 {
  uint32_t w[4];
};

__device__ __forceinline__ bf16x8 asBf16x8(const U128& v) { return __builtin_bit_cast(bf16x8, v); }

__device__ __forceinline__ U128 load16(const void* p) {
  return *reinterpret_cast<const U128*>(p);
}

__device__ __forceinline__ U128 zero16() {
  U128 z;
  z.w[0] = z.w[1] = z.w[2] = z.w[3] = 0;
  return z;
}

// Where the B operand (the skinny activation x) is read from.
struct XGlobal {
  const uint16_t* x;  // [M, K] row-major
  int64_t stride;     // elements between rows (K)
};
struct XLds {
  const uint16_t* x;  // LDS copy [16 * MB rows][stride], rows >= M are zero
  int stride;
};

template <int NF, int MB, int kWaves>
struct SkinnyCore {
  static constexpr int kTileN = 16 * NF;
  static constexpr int kTileM = 16 * MB;
  // LDS floats needed by reduce(): one partial tile per wave.
  static constexpr int kLdsFloats = kWaves * kTileN * kTileM;
  static constexpr int kUnroll = 4;  // 64-column steps per batch

  // One batch of operands in registers: weights always, x only when it comes from global.
  template <typename XSrc>
  struct Batch {
    U128 a[kUnroll][NF][2];
    U128 x[kUnroll][MB][2];
  };

  template <typename XSrc>
  __device__ static U128 loadX(const XSrc& xs, int b, int r, int g, int M, int64_t k) {
    const int m = b * 16 + r;
    if constexpr (__is_same(XSrc, XLds)) {
      return load16(xs.x + m * xs.stride + k + g * 8);
    } else {
      return m < M ? load16(xs.x + m * xs.stride + k + g * 8) : zero16();
    }
  }

  struct Rows {
    const uint16_t* w[NF];
    bool valid[NF];
  };

  __device__ static Rows rows(const uint16_t* w, int64_t N, int64_t K, int64_t n0, int r, int g) {
    Rows rw;
#pragma unroll
    for (int f = 0; f < NF; ++f) {
      const int64_t n = n0 + f * 16 + r;
      rw.valid[f] = n < N;
      rw.w[f] = w + (rw.valid[f] ? n : 0) * K + g * 8;
    }
    return rw;
  }

  // Issues the weight loads (and global x loads) of the batch starting at step s0.
  template <typename XSrc>
  __device__ static void issue(Batch<XSrc>& bt, const Rows& rw, const XSrc& xs, int M, int s0,
                               int step_end, int r, int g) {
#pragma unroll
    for (int u = 0; u < kUnroll; ++u) {
      const int s = s0 + u * kWaves;
      const bool live = s < step_end;
      const int64_t k0 = static_cast<int64_t>(live ? s : 0) * 64;
#pragma unroll
      for (int f = 0; f < NF; ++f) {
        bt.a[u][f][0] = (live && rw.valid[f]) ? load16(rw.w[f] + k0) : zero16();
        bt.a[u][f][1] = (live && rw.valid[f]) ? load16(rw.w[f] + k0 + 32) : zero16();
      }
      if constexpr (!__is_same(XSrc, XLds)) {
#pragma unroll
        for (int b = 0; b < MB; ++b) {
          bt.x[u][b][0] = live ? loadX(xs, b, r, g, M, k0) : zero16();
          bt.x[u][b][1] = live ? loadX(xs, b, r, g, M, k0 + 32) : zero16();
        }
      }
    }
  }

  template <typename XSrc>
  __device__ static void compute(f32x4 (&acc)[NF][MB], Batch<XSrc>& bt, const XSrc& xs, int M,
                                 int s0, int step_end, int r, int g) {
#pragma unroll
    for (int u = 0; u < kUnroll; ++u) {
      const int s = s0 + u * kWaves;
      if (s >= step_end) break;  // uniform per wave
      const int64_t k0 = static_cast<int64_t>(s) * 64;
#pragma unroll
      for (int h = 0; h < 2; ++h) {
        U128 bx[MB];
#pragma unroll
        for (int b = 0; b < MB; ++b) {
          if constexpr (__is_same(XSrc, XLds))
            bx[b] = loadX(xs, b, r, g, M, k0 + h * 32);
          else
            bx[b] = bt.x[u][b][h];
        }
#pragma unroll
        for (int f = 0; f < NF; ++f)
#pragma unroll
          for (int b = 0; b < MB; ++b)
            acc[f][b] = __builtin_amdgcn_mfma_f32_16x16x32_bf16(asBf16x8(bt.a[u][f][h]),
                                                                asBf16x8(bx[b]), acc[f][b], 0, 0, 0);
      }
    }
  }

  // Accumulates steps [step_begin, step_end) of the tile at weight row n0 and leaves the reduced
  // fp32 tile [kTileN][kTileM] in lds[0 .. tile). Wave w takes steps step_begin + w, + kWaves,
  // ...; batches are double-buffered (the next batch's loads are in flight while the current one
  // is multiplied). `prologue` runs once after the first batch's loads are issued (it may fill
  // the LDS copy of x and must end with __syncthreads()).
  template <typename XSrc, typename Prologue>
  __device__ static void run(const uint16_t* __restrict__ w, const XSrc& xs, int64_t N, int64_t K,
                             int M, int64_t n0, int step_begin, int step_end, float* lds,
                             Prologue&& prologue) {
    const int lane = threadIdx.x % kWave;
    const int wave = threadIdx.x / kWave;
    const int r = lane % 16, g = lane / 16;
    f32x4 acc[NF][MB];
#pragma unroll
    for (int f = 0; f < NF; ++f)
#pragma unroll
      for (int b = 0; b < MB; ++b) acc[f][b] = f32x4{0.f, 0.f, 0.f, 0.f};
    const Rows rw = rows(w, N, K, n0, r, g);
    constexpr int kStride = kUnroll * kWaves;
    Batch<XSrc> b0, b1;
    int s0 = step_begin + wave;
    issue(b0, rw, xs, M, s0, step_end, r, g);
    prologue();
    for (; s0 < step_end; s0 += 2 * kStride) {
      const int s1 = s0 + kStride;
      if (s1 < step_end) issue(b1, rw, xs, M, s1, step_end, r, g);
      compute(acc, b0, xs, M, s0, step_end, r, g);
      if (s1 >= step_end) break;
      const int s2 = s1 + kStride;
      if (s2 < step_end) issue(b0, rw, xs, M, s2, step_end, r, g);
      compute(acc, b1, xs, M, s1, step_end, r, g);
    }
    reduce(acc, lds, r, g, wave);
  }

  template <typename XSrc>
  __device__ static void run(const uint16_t* __restrict__ w, const XSrc& xs, int64_t N, int64_t K,
                             int M, int64_t n0, int step_begin, int step_end, float* lds) {
    run(w, xs, N, K, M, n0, step_begin, step_end, lds, [] {});
  }

  // Partial tiles -> LDS [wave][n][m], then a fixed-order sum over waves into lds[0..tile).
  __device__ static void reduce(f32x4 (&acc)[NF][MB], float* lds, int r, int g, int wave) {
    float* mine = lds + wave * kTileN * kTileM;
#pragma unroll
    for (int f = 0; f < NF; ++f)
#pragma unroll
      for (int b = 0; b < MB; ++b)
#pragma unroll
        for (int i = 0; i < 4; ++i) mine[(f * 16 + g * 4 + i) * kTileM + b * 16 + r] = acc[f][b][i];
    __syncthreads();
    for (int idx = threadIdx.x; idx < kTileN * kTileM; idx += blockDim.x) {
      float sum = lds[idx];
      for (int v = 1; v < kWaves; ++v) sum += lds[v * kTileN * kTileM + idx];
      lds[idx] = sum;
    }
    __syncthreads();
  }
};

// Split-K across workgroups. Every workgroup (tile, split) stores its partial tile to
// workspace; the last one to arrive for a tile (atomic ticket) sums all partials in split order
// — independent of arrival order — into lds and returns true; the others return false. The
// ticket is reset by that last workgroup, so counters are zero again after every launch.
//   partials: [tiles][splits][tile_elems] fp32, counters: [tiles] uint32 (zero before first use)
template <int kTileElems>
__device__ bool splitKReduce(float* lds, float* partials, uint32_t* counters, int tile, int split,
                             int splits) {
  if (splits <= 1) return true;
  float* mine = partials + (static_cast<int64_t>(tile) * splits + split) * kTileElems;
  for (int idx = threadIdx.x; idx < kTileElems; idx += blockDim.x) mine[idx] = lds[idx];
  __threadfence();
  __syncthreads();
  __shared__ uint32_t ticket;
  if (threadIdx.x == 0) ticket = atomicAdd(counters + tile, 1u);
  __syncthreads();
  if (ticket != static_cast<uint32_t>(splits - 1)) return false;
  __threadfence();
  const float* base = partials + static_cast<int64_t>(tile) * splits * kTileElems;
  for (int idx = threadIdx.x; idx < kTileElems; idx += blockDim.x) {
    float sum = 0.f;
    for (int s = 0; s < splits; ++s) sum += base[s * kTileElems + idx];
    lds[idx] = sum;
  }
  if (threadIdx.x == 0) counters[tile] = 0u;
  __syncthreads();
  return true;
}

// RMSNorm prologue: xs[m][0..K) = bf16(x[m] * rsqrt(mean(x[m]^2) + eps) * w) for m < M, zero rows
// for M <= m < rows. Wave w owns rows w, w + waves, ...; each lane holds up to kVec 16-byte
// pieces of every owned row in registers, so a row is read once and all rows of a wave are in
// flight together. Requires K % 8 == 0 and K <= 64 * 8 * kVec.
template <int kRowsPerWave, int kVec>
__device__ inline void rmsNormRowsToLds(const uint16_t* __restrict__ x, const uint16_t* __restrict__ w,
                                        int M, int rows, int K, float eps, uint16_t* xs,
                                        int stride) {
  const int lane = threadIdx.x % kWave;
  const int wave = threadIdx.x / kWave;
  const int waves = blockDim.x / kWave;
  const int vecs = K / 8;
  U128 raw[kRowsPerWave][kVec];
  U128 wv[kVec];
#pragma unroll
  for (int j = 0; j < kVec; ++j) {
    const int v = lane + j * kWave;
    wv[j] = v < vecs ? load16(w + v * 8) : zero16();
  }
#pragma unroll
  for (int i = 0; i < kRowsPerWave; ++i) {
    const int m = wave + i * waves;
#pragma unroll
    for (int j = 0; j < kVec; ++j) {
      const int v = lane + j * kWave;
      raw[i][j] = (m < M && v < vecs) ? load16(x + static_cast<int64_t>(m) * K + v * 8) : zero16();
    }
  }
#pragma unroll
  for (int i = 0; i < kRowsPerWave; ++i) {
    const int m = wave + i * waves;
    if (m >= rows) break;
    float sq = 0.f;
#pragma unroll
    for (int j = 0; j < kVec; ++j)
#pragma unroll
      for (int e = 0; e < 4; ++e) {
        const float lo = bf16ToFloat(raw[i][j].w[e] & 0xffffu), hi = bf16ToFloat(raw[i][j].w[e] >> 16);
        sq += lo * lo + hi * hi;
      }
    sq = waveSum(sq);
    const float inv = m < M ? 1.0f / sqrtf(sq / static_cast<float>(K) + eps) : 0.f;
    uint16_t* dst = xs + m * stride;
#pragma unroll
    for (int j = 0; j < kVec; ++j) {
      const int v = lane + j * kWave;
      if (v >= vecs) break;
      U128 out;
#pragma unroll
      for (int e = 0; e < 4; ++e) {
        const float lo = bf16ToFloat(raw[i][j].w[e] & 0xffffu) * inv * bf16ToFloat(wv[j].w[e] & 0xffffu);
        const float hi = bf16ToFloat(raw[i][j].w[e] >> 16) * inv * bf16ToFloat(wv[j].w[e] >> 16);
        out.w[e] = static_cast<uint32_t>(floatToBf16(lo)) | (static_cast<uint32_t>(floatToBf16(hi)) << 16);
      }
      *reinterpret_cast<U128*>(dst + v * 8) = out;
    }
  }
  __syncthreads();
}

}  // namespace dk
