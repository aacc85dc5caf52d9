#pragma once

// Weight-streaming MFMA core for skinny GEMMs on gfx950: out[m, n] = sum_k x[m, k] * w[n, k]
// with few rows m (decode batch, M <= 16 * MB) and a large bf16 weight w [N, K] read once.
//
// Work split
//   - A workgroup owns an N-tile of 16 * NF weight rows and a range of 64-column K steps (a
//     caller may split K over grid.y and reduce the partial tiles itself).
//   - Its kWaves waves take steps begin + wave, + kWaves, ...: per step a lane loads two 16-byte
//     runs of one weight row, so every wave-wide load pair covers 16 rows x 128 contiguous bytes
//     (whole cache lines, each byte fetched once). With kIdle > 0 the first kIdle waves take no
//     step (waves kIdle.. take begin + wave - kIdle, + kWaves - kIdle, ...): a gated caller's
//     polling wave then has no weight loads in flight, so its poll does not complete behind them
//     (a wave's loads complete in issue order).
//   - x fragments are loaded from global memory with the weights (x is small and stays in L2).
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

// 16 bytes as a native 4 x u32 vector: kept in 4 consecutive VGPRs, which is the register
// layout an MFMA operand needs, so no moves are required to feed it.
typedef uint32_t U128 __attribute__((ext_vector_type(4)));

__device__ __forceinline__ bf16x8 asBf16x8(const U128& v) { return __builtin_bit_cast(bf16x8, v); }

__device__ __forceinline__ U128 load16(const void* p) {
  return *reinterpret_cast<const U128*>(p);
}

__device__ __forceinline__ U128 zero16() { return U128{0u, 0u, 0u, 0u}; }

// 16 bytes of device memory (a global load whatever the compiler knows of p's origin).
__device__ __forceinline__ U128 gload16(const void* p) {
  return *gp(reinterpret_cast<const U128*>(p));
}

// Memory-access policies for activations.
//   PlainMem         ordinary loads and stores: the data crosses a kernel boundary (which makes
//                    writes visible to every XCD) before it is read.
//   WriteThroughMem  for data that other workgroups of the same launch read: stores are
//                    agent-scope (global_store ... sc1), written through to the coherent memory
//                    side instead of staying in this XCD's L2 (the L2s of the 8 XCDs are not
//                    coherent with each other); loads are plain. Plain loads are correct only
//                    for lines that no CU of the reading XCD has read earlier in the launch (a
//                    stale copy could hit), which the persistent decoder stack guarantees by
//                    giving every layer its own activation buffers. Plain loads let the XCD's
//                    L2 serve repeated reads of a line, where agent-scope loads would send every
//                    workgroup's request to the same memory channel.
struct PlainMem {
  __device__ __forceinline__ static U128 load16(const void* p) { return gload16(p); }
  __device__ __forceinline__ static uint16_t loadU16(const uint16_t* p) { return *gp(p); }
  __device__ __forceinline__ static void storeU16(uint16_t* p, uint16_t v) { *gp(p) = v; }
  __device__ __forceinline__ static void storeU32(uint32_t* p, uint32_t v) { *gp(p) = v; }
  __device__ __forceinline__ static void store16(void* p, U128 v) {
    *gp(reinterpret_cast<U128*>(p)) = v;
  }
};

struct WriteThroughMem {
  __device__ __forceinline__ static U128 load16(const void* p) { return gload16(p); }
  __device__ __forceinline__ static uint16_t loadU16(const uint16_t* p) { return *gp(p); }
  __device__ __forceinline__ static void storeU16(uint16_t* p, uint16_t v) {
    __hip_atomic_store(gp(p), v, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
  }
  __device__ __forceinline__ static void storeU32(uint32_t* p, uint32_t v) {
    __hip_atomic_store(gp(p), v, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
  }
  // 16 bytes with the same cache policy the agent-scope stores above get (sc1: written through
  // to the coherent memory side). The caller's s_waitcnt vmcnt(0) covers it like any store.
  __device__ __forceinline__ static void store16(void* p, U128 v) {
    asm volatile("global_store_dwordx4 %0, %1, off sc1" : : "v"(p), "v"(v) : "memory");
  }
};

// Element (m, k) of an activation [rows, 64 * steps] stored in MFMA fragment order: blocks of
// [16 rows x 32 columns], one per (row block b, 64-column step s, half h), each laid out as
// [column group g = 8 columns][row r][8 columns]. A fragment load of (b, s, h), where lane
// g * 16 + r reads row 16 b + r, columns 64 s + 32 h + 8 g .. + 7, is then one contiguous 1 KB
// read (the row-major [rows, K] layout spreads it over 16 rows: 64 bytes of each of 16 lines,
// measured 2.7 times slower for a 57 KB activation). Rows are padded to whole 16-row blocks.
__device__ __forceinline__ int64_t fragOffset(int m, int64_t k, int steps) {
  const int64_t b = m >> 4, r = m & 15, s = k >> 6, h = (k >> 5) & 1, g = (k >> 3) & 3;
  return ((((b * steps + s) * 2 + h) * 4 + g) * 16 + r) * 8 + (k & 7);
}

// Offset of element (m, k) of an activation with `ld` columns: row-major when frag_steps is 0,
// else fragment order with frag_steps = ld / 64 (fragOffset).
__device__ __forceinline__ int64_t actOffset(int m, int64_t k, int64_t ld, int frag_steps) {
  return frag_steps > 0 ? fragOffset(m, k, frag_steps) : m * ld + k;
}

// The B operand (the skinny activation x): [M, K] row-major with `stride` elements per row.
struct XGlobal {
  const uint16_t* x;
  int64_t stride;
};

// The B operand in fragment order (fragOffset) with `steps` = K / 64, rows padded to 16-row
// blocks. A separate type, so the layout is fixed at compile time in each GEMM.
struct XFrag {
  const uint16_t* x;
  int steps;
};

// kUnroll: 64-column steps per batch and wave (two batches are in flight); kIdle: leading waves
// without steps (their partial tiles are zero).
template <int NF, int MB, int kWaves, int kUnroll = 4, int kIdle = 0>
struct SkinnyCore {
  static_assert(kIdle >= 0 && kIdle < kWaves, "at least one wave takes steps");
  static constexpr int kCW = kWaves - kIdle;  // waves that take steps
  static constexpr int kTileN = 16 * NF;
  static constexpr int kTileM = 16 * MB;
  // LDS floats needed by reduce() or storePartials(): one partial tile per wave (rows padded to
  // kTileM + 1 floats by storePartials).
  static constexpr int kPadM = kTileM + 1;
  static constexpr int kLdsFloats = kWaves * kTileN * kPadM;

  struct WBatch {
    U128 a[kUnroll][NF][2];
  };
  struct XBatch {
    U128 x[kUnroll][MB][2];
  };

  // Row pointers of this lane (row r of each 16-row block, columns from g * 8). Rows past N
  // (weights) or M (x) are clamped to the last valid row: their loads stay in bounds and the
  // products land only in output rows and columns the epilogues discard, so the loads need no
  // per-lane predicate.
  struct Rows {
    const uint16_t* w[NF];
  };

  __device__ __forceinline__ static Rows rows(const uint16_t* w, int64_t N, int64_t K, int64_t n0,
                                              int r, int g) {
    Rows rw;
#pragma unroll
    for (int f = 0; f < NF; ++f) {
      const int64_t n = n0 + f * 16 + r;
      rw.w[f] = w + (n < N ? n : N - 1) * K + g * 8;
    }
    return rw;
  }

  // Lane pointers of each row block; kStep and kHalf are the element distances of a 64-column
  // step and of the second 32-column half of a step in the layout.
  template <bool kFrag>
  struct XRowsT {
    static constexpr int64_t kStep = kFrag ? 1024 : 64;
    static constexpr int64_t kHalf = kFrag ? 512 : 32;
    const uint16_t* x[MB];
  };
  using XRows = XRowsT<false>;

  __device__ __forceinline__ static XRows xrows(const XGlobal& xs, int M, int r, int g) {
    XRows xr;
#pragma unroll
    for (int b = 0; b < MB; ++b) {
      const int m = b * 16 + r;
      xr.x[b] = xs.x + static_cast<int64_t>(m < M ? m : M - 1) * xs.stride + g * 8;
    }
    return xr;
  }

  // Fragment order: padded rows are read as they are (they feed discarded outputs only).
  __device__ __forceinline__ static XRowsT<true> xrows(const XFrag& xs, int, int r, int g) {
    XRowsT<true> xr;
#pragma unroll
    for (int b = 0; b < MB; ++b)
      xr.x[b] = xs.x + (static_cast<int64_t>(b) * xs.steps * 128 + g * 16 + r) * 8;
    return xr;
  }

  // Weight loads of the batch whose first step is s0 (steps s0 + u * kCW). s0 is uniform
  // over the wave, so steps past step_end are skipped with a scalar branch; their registers are
  // never read (compute stops at step_end).
  __device__ __forceinline__ static void issueW(WBatch& bt, const Rows& rw, int s0, int step_end) {
#pragma unroll
    for (int u = 0; u < kUnroll; ++u) {
      const int s = s0 + u * kCW;
      if (s >= step_end) break;
      const int64_t k0 = static_cast<int64_t>(s) * 64;
#pragma unroll
      for (int f = 0; f < NF; ++f) {
        bt.a[u][f][0] = gload16(rw.w[f] + k0);
        bt.a[u][f][1] = gload16(rw.w[f] + k0 + 32);
      }
    }
  }

  // x loads of the same batch.
  template <class Mem = PlainMem, bool kFrag = false>
  __device__ __forceinline__ static void issueX(XBatch& bt, const XRowsT<kFrag>& xr, int s0,
                                                int step_end) {
#pragma unroll
    for (int u = 0; u < kUnroll; ++u) {
      const int s = s0 + u * kCW;
      if (s >= step_end) break;
      const int64_t k0 = static_cast<int64_t>(s) * XRowsT<kFrag>::kStep;
#pragma unroll
      for (int b = 0; b < MB; ++b) {
        bt.x[u][b][0] = Mem::load16(xr.x[b] + k0);
        bt.x[u][b][1] = Mem::load16(xr.x[b] + k0 + XRowsT<kFrag>::kHalf);
      }
    }
  }

  __device__ __forceinline__ static void compute(f32x4 (&acc)[NF][MB], const WBatch& wb,
                                                 const XBatch& xb, int s0, int step_end) {
#pragma unroll
    for (int u = 0; u < kUnroll; ++u) {
      if (s0 + u * kCW >= step_end) break;  // uniform per wave
#pragma unroll
      for (int h = 0; h < 2; ++h)
#pragma unroll
        for (int f = 0; f < NF; ++f)
#pragma unroll
          for (int b = 0; b < MB; ++b)
            acc[f][b] = __builtin_amdgcn_mfma_f32_16x16x32_bf16(asBf16x8(wb.a[u][f][h]),
                                                                asBf16x8(xb.x[u][b][h]), acc[f][b],
                                                                0, 0, 0);
    }
  }

  __device__ __forceinline__ static void zero(f32x4 (&acc)[NF][MB]) {
#pragma unroll
    for (int f = 0; f < NF; ++f)
#pragma unroll
      for (int b = 0; b < MB; ++b) acc[f][b] = f32x4{0.f, 0.f, 0.f, 0.f};
  }

  // Accumulates steps [step_begin, step_end) of the tile at weight row n0 and leaves the reduced
  // fp32 tile [kTileN][kTileM] in lds[0 .. tile). Batches are double-buffered: the next batch's
  // loads are in flight while the current one is multiplied.
  __device__ __forceinline__ static void run(const uint16_t* __restrict__ w, const XGlobal& xs,
                                             int64_t N, int64_t K, int M, int64_t n0,
                                             int step_begin, int step_end, float* lds) {
    const int lane = freshThreadIdx() % kWave;
    const int wave = __builtin_amdgcn_readfirstlane(threadIdx.x / kWave);
    const int r = lane % 16, g = lane / 16;
    f32x4 acc[NF][MB];
    zero(acc);
    const Rows rw = rows(w, N, K, n0, r, g);
    const XRows xr = xrows(xs, M, r, g);
    constexpr int kStride = kUnroll * kCW;
    WBatch w0, w1;
    XBatch x0, x1;
    int s0 = wave < kIdle ? step_end : step_begin + wave - kIdle;  // uniform
    issueW(w0, rw, s0, step_end);
    issueX(x0, xr, s0, step_end);
    for (; s0 < step_end; s0 += 2 * kStride) {
      const int s1 = s0 + kStride;
      if (s1 < step_end) {
        issueW(w1, rw, s1, step_end);
        issueX(x1, xr, s1, step_end);
      }
      compute(acc, w0, x0, s0, step_end);
      if (s1 >= step_end) break;
      const int s2 = s1 + kStride;
      if (s2 < step_end) {
        issueW(w0, rw, s2, step_end);
        issueX(x0, xr, s2, step_end);
      }
      compute(acc, w1, x1, s1, step_end);
    }
    reduce(acc, lds, r, g, wave);
  }

  // run() for an x that another workgroup of the same launch produces: the first two weight
  // batches are requested, then gate() (called by every thread) waits until x is ready, and only
  // then are the x batches loaded (with Mem). The batches are accumulated in the order run()
  // uses, so both give bit-identical tiles.
  // mark(0) (every thread calls it) marks the point where the tile is reduced, mark(1) the point
  // where the first x batches are requested. xs: XGlobal (row-major) or XFrag (fragment order).
  template <class Mem, class Gate, class Mark = NoMark, class XS = XGlobal>
  __device__ __forceinline__ static void runGated(const uint16_t* __restrict__ w, const XS& xs,
                                                  int64_t N, int64_t K, int M, int64_t n0,
                                                  int step_begin, int step_end, float* lds,
                                                  Gate&& gate, Mark mark = Mark{}) {
    const int lane = freshThreadIdx() % kWave;
    const int wave = __builtin_amdgcn_readfirstlane(threadIdx.x / kWave);
    const int r = lane % 16, g = lane / 16;
    f32x4 acc[NF][MB];
    zero(acc);
    const Rows rw = rows(w, N, K, n0, r, g);
    const auto xr = xrows(xs, M, r, g);
    constexpr int kStride = kUnroll * kCW;
    WBatch w0, w1;
    XBatch x0, x1;
    int s0 = wave < kIdle ? step_end : step_begin + wave - kIdle;  // uniform
    issueW(w0, rw, s0, step_end);
    if (s0 + kStride < step_end) issueW(w1, rw, s0 + kStride, step_end);
    gate();
    issueX<Mem>(x0, xr, s0, step_end);
    if (s0 + kStride < step_end) issueX<Mem>(x1, xr, s0 + kStride, step_end);
    mark(1);  // loads of the first batches issued (a tracing caller may wait for them here)
    for (; s0 < step_end; s0 += 2 * kStride) {
      const int s1 = s0 + kStride;
      compute(acc, w0, x0, s0, step_end);
      if (s1 >= step_end) break;
      const int s2 = s1 + kStride;
      if (s2 < step_end) {
        issueW(w0, rw, s2, step_end);
        issueX<Mem>(x0, xr, s2, step_end);
      }
      compute(acc, w1, x1, s1, step_end);
      const int s3 = s2 + kStride;
      if (s3 < step_end) {
        issueW(w1, rw, s3, step_end);
        issueX<Mem>(x1, xr, s3, step_end);
      }
    }
    reduce(acc, lds, r, g, wave);
    mark(0);
  }

  // Partial tiles -> LDS [wave][n][m], then a fixed-order sum over waves into lds[0..tile).
  // reduce() without its sum: each wave's partial tile stays in its slice of lds (wave w at
  // lds + w * kTileN * kPadM, row n at n * kPadM: rows padded so that an epilogue walking n
  // across lanes spreads over the LDS banks), for an epilogue that reads every element once and
  // adds the slices itself (partialSum, in reduce()'s order), which saves reduce()'s second
  // pass over LDS and its second barrier.
  __device__ __forceinline__ static void storePartials(f32x4 (&acc)[NF][MB], float* lds, int r,
                                                       int g, int wave) {
    float* mine = lds + wave * kTileN * kPadM;
#pragma unroll
    for (int f = 0; f < NF; ++f)
#pragma unroll
      for (int b = 0; b < MB; ++b)
#pragma unroll
        for (int i = 0; i < 4; ++i) mine[(f * 16 + g * 4 + i) * kPadM + b * 16 + r] = acc[f][b][i];
    __syncthreads();
  }
  // element (n, m) of the tile: row n (weight row), column m (batch row)
  __device__ __forceinline__ static float partialSum(const float* lds, int n, int m) {
    float sum = lds[n * kPadM + m];
#pragma unroll
    for (int v = 1; v < kWaves; ++v) sum += lds[(v * kTileN + n) * kPadM + m];
    return sum;
  }

  __device__ __forceinline__ static void reduce(f32x4 (&acc)[NF][MB], float* lds, int r, int g,
                                                int wave) {
    float* mine = lds + wave * kTileN * kTileM;
#pragma unroll
    for (int f = 0; f < NF; ++f)
#pragma unroll
      for (int b = 0; b < MB; ++b)
#pragma unroll
        for (int i = 0; i < 4; ++i) mine[(f * 16 + g * 4 + i) * kTileM + b * 16 + r] = acc[f][b][i];
    __syncthreads();
    for (int idx = freshThreadIdx(); idx < kTileN * kTileM; idx += kWaves * kWave) {
      float sum = lds[idx];
      for (int v = 1; v < kWaves; ++v) sum += lds[v * kTileN * kTileM + idx];
      lds[idx] = sum;
    }
    __syncthreads();
  }
};

}  // namespace dk
