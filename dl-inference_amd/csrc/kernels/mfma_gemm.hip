// MFMA GEMMs of the generic operators on gfx950 (linear, matmul and conv2d for many rows; decode
// sizes use the weight-streaming kernels of gemm.hip / decode.hip).
//
//   C[r, c] = sum_k A(r, k) * B(c, k), then an epilogue per output element (bias, ReLU, layout)
//
//  mfma_linear_f32_<t>      fp32: A = x [M, K], B = w [N, K] (linear/kernel.py:6-44), or
//  mfma_matmul_f32          B = b [K, N] (matmul/kernel.py:6-40); fp32 MFMA 16x16x4
//  mfma_conv2d_f32          im2col-free conv2d (conv2d/kernel.py:6-49): A = weight [OC, C*KH*KW]
//                           rows, B = the input patch of each output pixel, gathered from NCHW
//                           x while staging (never materialised); out NCHW, optional fused ReLU
//  mfma_linear_bf16_<t>     bf16 x, w (K % 8 == 0), bf16 MFMA 16x16x32, fp32 accumulation,
//                           bf16 or fp32 out, optional ReLU
//  mfma_linear_residual_bf16_<t>  the same plus a residual add (bf16 out)
//  mfma_gate_up_silu_bf16_<t>     the same over an interleaved gate/up weight, SwiGLU epilogue
//  mfma_linear_f32_splitk   fp32 linear / conv2d with K split over grid.z into a workspace,
//  mfma_conv2d_f32_splitk   then a fixed-order sum with bias and ReLU (splitk_reduce_f32,
//                           conv_splitk_reduce_f32)
//
// Work split: a 256-thread workgroup owns a BM x BN tile of C (4 waves, 2 x 2, each BM/2 x BN/2
// as 16 x 16 MFMA tiles) and walks K in BK-wide slices. A slice of A and B is loaded from global
// memory into registers (coalesced: consecutive lanes take consecutive k of a row, or
// consecutive rows/pixels when those are contiguous in memory), written to LDS as [row][k] with
// a padded row pitch, and read back as MFMA fragments; the next slice's loads are in flight
// while the current one is multiplied (the bf16 GEMM keeps two slices in flight and two LDS
// buffers, and orders its tiles by XCD: see the bf16 core). Rows, columns and k past the ends
// load zeros (or, in the bf16 GEMM, clamped rows whose results are dropped), so any shape works.
// Every output is a fixed-order sum: results do not depend on timing.
//
// Conv output pixels are the C columns, so the 16 lanes that share an output row of an MFMA
// tile store 16 consecutive pixels of one channel (coalesced NCHW stores).
#include "common.h"
#include "skinny.h"

using namespace dk;

namespace {

constexpr int kGemmThreads = 256;

// ---- operand sources -------------------------------------------------------------------------
// load(row, k): element (row, k) as fp32, zero outside [0, rows) x [0, K). kFastK: consecutive k
// of a row are adjacent in memory (else consecutive rows are).

struct RowsK {  // p[row * ld + k]
  static constexpr bool kFastK = true;
  const float* p;
  int64_t rows, K, ld;
  __device__ __forceinline__ float load(int64_t row, int64_t k) const {
    return row < rows && k < K ? gp(p)[row * ld + k] : 0.f;
  }
};

struct KRows {  // p[k * ld + row] (matmul's b [K, N])
  static constexpr bool kFastK = false;
  const float* p;
  int64_t rows, K, ld;
  __device__ __forceinline__ float load(int64_t row, int64_t k) const {
    return row < rows && k < K ? gp(p)[k * ld + row] : 0.f;
  }
};

// Source hooks used by gemmF32 (no-ops for the plain layouts): begin() once per workgroup,
// prepare() for every K slice before it is fetched (threads < BK fill a per-slice table),
// load(row, k, kl, tab) with kl = k - slice start.
struct NoTable {
  __device__ __forceinline__ void begin(int64_t, int, int) {}
  template <int BK>
  __device__ __forceinline__ void prepareT(int64_t, int, int2*) const {}
};

struct RowsKT : RowsK, NoTable {
  __device__ __forceinline__ float load(int64_t row, int64_t k, int, const int2*) const {
    return RowsK::load(row, k);
  }
};

struct KRowsT : KRows, NoTable {
  __device__ __forceinline__ float load(int64_t row, int64_t k, int, const int2*) const {
    return KRows::load(row, k);
  }
};

// Input patch of a zero-padded NCHW conv: column `row` = output pixel (n, oy, ox), k = (c, ky,
// kx) over k_base + [0, K). The tile's columns are fixed per thread (row = c0 + t % BN), so
// begin() decomposes the pixel once; prepare() tabulates (c * H * W + ky * W + kx, ky, kx) for
// the BK k of a slice, and a load is a table read, two bounds checks and one gather. 32-bit
// index math (the host checks that every index fits).
struct ConvPatch {
  static constexpr bool kFastK = false;
  const float* x;
  int rows, K, k_base, C, H, W, KH, KW, OH, OW, SH, SW, PH, PW;
  bool valid = false;
  int iy0 = 0, ix0 = 0, base = 0;
  __device__ __forceinline__ void begin(int64_t c0, int t, int bn) {
    const int pixel = static_cast<int>(c0) + t % bn;
    valid = pixel < rows;
    const int ox = pixel % OW, q = pixel / OW;
    const int oy = q % OH, n = q / OH;
    iy0 = oy * SH - PH;
    ix0 = ox * SW - PW;
    base = n * C * H * W + iy0 * W + ix0;
  }
  template <int BK>
  __device__ __forceinline__ void prepareT(int64_t k0, int t, int2* tab) const {
    const int k = static_cast<int>(k0) + t;
    if (t < BK && k < K) {
      const int kk = k_base + k, khw = KH * KW;
      const int c = kk / khw, rem = kk - c * khw;
      const int ky = rem / KW, kx = rem - ky * KW;
      tab[t] = int2{(c * H + ky) * W + kx, (ky << 16) | kx};
    }
  }
  __device__ __forceinline__ float load(int64_t, int64_t k, int kl, const int2* tab) const {
    if (!valid || k >= K) return 0.f;
    const int2 e = tab[kl];
    const int iy = iy0 + (e.y >> 16), ix = ix0 + (e.y & 0xFFFF);
    if (iy < 0 || iy >= H || ix < 0 || ix >= W) return 0.f;
    return gp(x)[base + e.x];
  }
};

// ---- tile order ----------------------------------------------------------------------------------
// Workgroups are handed to the 8 XCDs round robin by linear id, so XCD x gets the x-th contiguous
// range of tiles of a grouped order (kGroupRows row blocks per group, row blocks fastest): the
// tiles one XCD runs at once share A row blocks and B column blocks in its L2. (gridDim.x, y) =
// (column tiles, row tiles); each blockIdx.z slice (a K split) is mapped the same way. At
// 8192 x 896 x 4864 (down_proj over a 4 x 2048 prompt) this took the bf16 GEMM from 110 to
// 79 us; with the plain order, the 7 column tiles of a row block ran on 7 XCDs, each fetching
// the row block from memory.
constexpr int kGroupRows = 8;

__device__ __forceinline__ void groupedTile(int BM, int BN, int64_t& r0, int64_t& c0) {
  const uint64_t nn = gridDim.x, nm = gridDim.y, T = nn * nm;
  const uint64_t L = blockIdx.x + nn * blockIdx.y;
  const uint64_t x = L % 8, l = L / 8;
  const uint64_t g = x * (T / 8) + (x < T % 8 ? x : T % 8) + l;  // a bijection of [0, T)
  const uint64_t per = kGroupRows * nn, grp = g / per, first = grp * kGroupRows;
  const uint64_t gs = nm - first < kGroupRows ? nm - first : kGroupRows;
  const uint64_t in = g - grp * per;
  r0 = static_cast<int64_t>(first + in % gs) * BM;
  c0 = static_cast<int64_t>(in / gs) * BN;
}

// ---- fp32 core ---------------------------------------------------------------------------------
// v_mfma_f32_16x16x4_f32: lane l supplies A[l % 16][kk] and B[kk][l % 16] for the step's k
// index kk = l / 16 and receives D[(l / 16) * 4 + i][l % 16], i < 4.
// LDS layout of one operand's K slice, chosen by how the source is staged:
//   kFastK (lanes take consecutive k of a row): [row][k], pitch BK + 4 floats (16-byte aligned
//     rows whose starts fall in distinct banks for the 16 rows of a fragment read), and a
//     lane's 4 consecutive k come in one 16-byte read;
//   otherwise (lanes take consecutive rows): [k][row], pitch ROWS + 2, so the stash writes
//     consecutive words and the four lane groups of a fragment read (k 8 apart) start 16
//     banks apart; 4 single reads.
template <bool kFastK, int ROWS, int BK>
struct SliceLayout {
  static constexpr int kPitch = kFastK ? BK + 4 : ROWS + 2;
  static constexpr int kFloats = kFastK ? ROWS * kPitch : BK * kPitch;
  __device__ __forceinline__ static int at(int row, int k) {
    return kFastK ? row * kPitch + k : k * kPitch + row;
  }
  // x[row][k .. k + 3], k a multiple of 4
  __device__ __forceinline__ static float4 four(const float* x, int row, int k) {
    if constexpr (kFastK) {
      return *reinterpret_cast<const float4*>(&x[at(row, k)]);
    } else {
      return float4{x[at(row, k)], x[at(row, k + 1)], x[at(row, k + 2)], x[at(row, k + 3)]};
    }
  }
};

template <int BM, int BN, class ASrc, class BSrc, class Epi>
__device__ __forceinline__ void gemmF32(ASrc A, BSrc B, int64_t R, int64_t Cn, int64_t K,
                                        const Epi& epi) {
  // 32-wide K slices (64 measured no faster on the CNN layers and wastes half a slice when K is
  // small).
  constexpr int BK = 32;
  using LA = SliceLayout<ASrc::kFastK, BM, BK>;
  using LB = SliceLayout<BSrc::kFastK, BN, BK>;
  constexpr int TM = BM / 32, TN = BN / 32;
  constexpr int AE = BM * BK / kGemmThreads, BE = BN * BK / kGemmThreads;
  __shared__ __attribute__((aligned(16))) float As[LA::kFloats];
  __shared__ __attribute__((aligned(16))) float Bs[LB::kFloats];
  const int t = threadIdx.x, lane = t % kWave, wave = t / kWave;
  const int wr = wave / 2, wc = wave % 2;
  int64_t r0, c0;
  groupedTile(BM, BN, r0, c0);
  __shared__ int2 ktab[2][BK];  // per-slice k table of a source that has one (double-buffered)
  float ra[AE], rb[BE];
  auto slot = [&](int e, int rows_in_tile, bool fast_k, int& row, int& k) {
    if (fast_k) {
      row = e / BK;
      k = e % BK;
    } else {
      row = e % rows_in_tile;
      k = e / rows_in_tile;
    }
  };
  auto fetch = [&](int64_t k0, const int2* tab) {
#pragma unroll
    for (int i = 0; i < AE; ++i) {
      int row, k;
      slot(t + i * kGemmThreads, BM, ASrc::kFastK, row, k);
      ra[i] = A.load(r0 + row, k0 + k, k, tab);
    }
#pragma unroll
    for (int i = 0; i < BE; ++i) {
      int row, k;
      slot(t + i * kGemmThreads, BN, BSrc::kFastK, row, k);
      rb[i] = B.load(c0 + row, k0 + k, k, tab);
    }
  };
  auto prepare = [&](int64_t k0, int2* tab) { B.template prepareT<BK>(k0, t, tab); };
  auto stash = [&] {
#pragma unroll
    for (int i = 0; i < AE; ++i) {
      int row, k;
      slot(t + i * kGemmThreads, BM, ASrc::kFastK, row, k);
      As[LA::at(row, k)] = ra[i];
    }
#pragma unroll
    for (int i = 0; i < BE; ++i) {
      int row, k;
      slot(t + i * kGemmThreads, BN, BSrc::kFastK, row, k);
      Bs[LB::at(row, k)] = rb[i];
    }
  };
  f32x4 acc[TM][TN];
#pragma unroll
  for (int i = 0; i < TM; ++i)
#pragma unroll
    for (int j = 0; j < TN; ++j) acc[i][j] = f32x4{0.f, 0.f, 0.f, 0.f};
  const int fr = lane % 16, fk = lane / 16;
  A.begin(r0, t, BM);
  B.begin(c0, t, BN);
  prepare(0, ktab[0]);
  __syncthreads();
  fetch(0, ktab[0]);
  int slice = 0;
  for (int64_t k0 = 0; k0 < K; k0 += BK, ++slice) {
    // the table of slice + 1 goes to the buffer that slice - 1's fetch read two barriers ago
    if (k0 + BK < K) prepare(k0 + BK, ktab[(slice + 1) & 1]);
    __syncthreads();  // every wave is done reading the previous slice
    stash();
    __syncthreads();
    if (k0 + BK < K) fetch(k0 + BK, ktab[(slice + 1) & 1]);
    // In each 32-k half of a slice, MFMA step s uses k = fk * 8 + s for lane group fk (A and B
    // alike, so each step is still a 4-term slice of the dot products).
#pragma unroll
    for (int kh = 0; kh < BK / 32; ++kh) {
      float4 a4[TM][2], b4[TN][2];
#pragma unroll
      for (int i = 0; i < TM; ++i)
#pragma unroll
        for (int h = 0; h < 2; ++h)
          a4[i][h] = LA::four(As, wr * (BM / 2) + i * 16 + fr, kh * 32 + fk * 8 + h * 4);
#pragma unroll
      for (int j = 0; j < TN; ++j)
#pragma unroll
        for (int h = 0; h < 2; ++h)
          b4[j][h] = LB::four(Bs, wc * (BN / 2) + j * 16 + fr, kh * 32 + fk * 8 + h * 4);
#pragma unroll
      for (int s = 0; s < 8; ++s)
#pragma unroll
        for (int i = 0; i < TM; ++i)
#pragma unroll
          for (int j = 0; j < TN; ++j)
            acc[i][j] = __builtin_amdgcn_mfma_f32_16x16x4f32(
                a4[i][s / 4][s % 4], b4[j][s / 4][s % 4], acc[i][j], 0, 0, 0);
    }
  }
  if constexpr (Epi::kPairs) {
    // column blocks 2 p and 2 p + 1 (16 wide) of a wave's tile go to one epi.pair call: the
    // C columns of an interleaved [gate 16 | up 16] weight pair up in the same lane
    static_assert(TN % 2 == 0, "column block pairs");
#pragma unroll
    for (int i = 0; i < TM; ++i)
#pragma unroll
      for (int j = 0; j < TN; j += 2)
#pragma unroll
        for (int v = 0; v < 4; ++v) {
          const int64_t row = r0 + wr * (BM / 2) + i * 16 + fk * 4 + v;
          const int64_t col = c0 + wc * (BN / 2) + j * 16 + fr;
          if (row < R && col + 16 < Cn) epi.pair(row, col, acc[i][j][v], acc[i][j + 1][v]);
        }
  } else {
#pragma unroll
    for (int i = 0; i < TM; ++i)
#pragma unroll
      for (int j = 0; j < TN; ++j)
#pragma unroll
        for (int v = 0; v < 4; ++v) {
          const int64_t row = r0 + wr * (BM / 2) + i * 16 + fk * 4 + v;
          const int64_t col = c0 + wc * (BN / 2) + j * 16 + fr;
          if (row < R && col < Cn) epi(row, col, acc[i][j][v]);
        }
  }
}

// ---- bf16 core ---------------------------------------------------------------------------------
// v_mfma_f32_16x16x32_bf16: lane l supplies A[l % 16][(l / 16) * 8 + j] and
// B[(l / 16) * 8 + j][l % 16], j < 8. Operands are [rows, K] row-major with K % 8 == 0 and
// 16-byte aligned rows, loaded 8 elements at a time.
//
// Pipeline (one 64-wide K slice per step): the slice being multiplied sits in one of two LDS
// buffers, the next one is written into the other from registers loaded two steps earlier, and
// the loads for the slice after that go out into the registers just written, all interleaved
// with the MFMAs (sched_group_barrier: one LDS read, or one LDS write and one global load, per two
// MFMAs; one per MFMA measured 15% slower on the 8192 x 9728 x 896 gate_up and 10% on down_proj),
// with one barrier per step. LDS rows hold 8 16-byte
// chunks, chunk c of row r at position c ^ ((r >> 1) & 7): the 16 lanes of a fragment read
// (rows r..r+15, one chunk) and the 16 lanes of a stash write (two rows) then fall on 16
// different 4-bank groups of the 64 banks (no conflicts; SQ_LDS_BANK_CONFLICT reads 0).
//
// Tiles in the XCD-grouped order (groupedTile).

// ld: row stride of a and b in elements (K for whole rows; a split-K part passes a and b offset
// to its first column, its own K and the full row stride).
// BK: K columns per slice, 64 or 128 (128 doubles the bytes each workgroup has in flight: the
// decode-sized kernels, whose few workgroups stream the weights).
// kStreamB: b (the weights) is read with nontemporal loads, for the decode-sized kernels, whose
// single row tile reads every weight once (many row tiles re-read them and keep cached loads).
// Each load instruction covers whole 128-byte lines (16 lanes per 256-byte row slice of a
// 128-wide slice); a streaming probe over 1 GiB read 6.5-6.9 TB/s that way against 5.8-6.0 with
// cached loads.
template <int BM, int BN, int BK = 64, bool kStreamB = false, class Epi>
__device__ __forceinline__ void gemmBf16(const uint16_t* a, const uint16_t* b, int64_t R,
                                         int64_t Cn, int64_t K, int64_t ld, const Epi& epi) {
  static_assert(BK == 64 || BK == 128, "slice width");
  constexpr int TM = BM / 32, TN = BN / 32;
  constexpr int VPR = BK / 8;  // 16-byte chunks per tile row
  constexpr int AV = BM * VPR / kGemmThreads, BV = BN * VPR / kGemmThreads;
  // the two operand buffers, then (after the last slice) the fp32 accumulator tile of the
  // epilogue, row pitch BN + 4 floats (the 4 row groups of an MFMA tile store land 16 banks apart)
  constexpr int CP = BN + 4;
  constexpr int kOperandBytes = 2 * (BM + BN) * BK * 2, kTileBytes = BM * CP * 4;
  __shared__ __attribute__((aligned(16)))
  uint8_t smem[kOperandBytes > kTileBytes ? kOperandBytes : kTileBytes];
  uint16_t* const As0 = reinterpret_cast<uint16_t*>(smem);
  uint16_t* const Bs0 = As0 + BM * BK;
  uint16_t* const As1 = Bs0 + BN * BK;
  uint16_t* const Bs1 = As1 + BM * BK;
  const int t = threadIdx.x, lane = t % kWave, wave = t / kWave;
  const int wr = wave / 2, wc = wave % 2;
  int64_t r0, c0;
  groupedTile(BM, BN, r0, c0);
  // 64-wide slices: rows of 128 bytes, two rows fill the 64 banks, chunk c at c ^ ((r >> 1) & 7);
  // 128-wide: rows of 256 bytes, chunk c of 16 at c ^ (r & 15)
  auto at = [](int row, int c) {
    return row * BK + (BK == 64 ? c ^ ((row >> 1) & 7) : c ^ (row & 15)) * 8;
  };
  // the thread's source rows, clamped into range (a clamped row loads a real row whose results
  // the epilogue drops); k past K loads zeros, in the last slice only
  const uint16_t* pa[AV];
  const uint16_t* pb[BV];
  const int kc = (t % VPR) * 8;
#pragma unroll
  for (int i = 0; i < AV; ++i) {
    const int64_t row = r0 + (t + i * kGemmThreads) / VPR;
    pa[i] = a + (row < R ? row : R - 1) * ld + kc;
  }
#pragma unroll
  for (int i = 0; i < BV; ++i) {
    const int64_t row = c0 + (t + i * kGemmThreads) / VPR;
    pb[i] = b + (row < Cn ? row : Cn - 1) * ld + kc;
  }
  auto loadB = [](const uint16_t* p) {
    if constexpr (kStreamB)
      return __builtin_nontemporal_load(gp(reinterpret_cast<const U128*>(p)));
    else
      return gload16(p);
  };
  auto fetch = [&](U128 (&xa)[AV], U128 (&xb)[BV], int64_t k0) {
    if (k0 + BK <= K) {
#pragma unroll
      for (int i = 0; i < AV; ++i) xa[i] = gload16(pa[i] + k0);
#pragma unroll
      for (int i = 0; i < BV; ++i) xb[i] = loadB(pb[i] + k0);
    } else {
      const bool in = k0 + kc < K;
#pragma unroll
      for (int i = 0; i < AV; ++i) xa[i] = in ? gload16(pa[i] + k0) : zero16();
#pragma unroll
      for (int i = 0; i < BV; ++i) xb[i] = in ? loadB(pb[i] + k0) : zero16();
    }
  };
  auto fetchWhole = [&](U128 (&xa)[AV], U128 (&xb)[BV], int64_t k0) {
#pragma unroll
    for (int i = 0; i < AV; ++i) xa[i] = gload16(pa[i] + k0);
#pragma unroll
    for (int i = 0; i < BV; ++i) xb[i] = loadB(pb[i] + k0);
  };
  auto stash = [&](const U128 (&xa)[AV], const U128 (&xb)[BV], uint16_t* as, uint16_t* bs) {
#pragma unroll
    for (int i = 0; i < AV; ++i) {
      const int e = t + i * kGemmThreads;
      *reinterpret_cast<U128*>(&as[at(e / VPR, e % VPR)]) = xa[i];
    }
#pragma unroll
    for (int i = 0; i < BV; ++i) {
      const int e = t + i * kGemmThreads;
      *reinterpret_cast<U128*>(&bs[at(e / VPR, e % VPR)]) = xb[i];
    }
  };
  f32x4 acc[TM][TN];
#pragma unroll
  for (int i = 0; i < TM; ++i)
#pragma unroll
    for (int j = 0; j < TN; ++j) acc[i][j] = f32x4{0.f, 0.f, 0.f, 0.f};
  const int fr = lane % 16, fk = lane / 16;
  auto frags = [&](const uint16_t* as, const uint16_t* bs, int s, U128 (&fa)[TM],
                   U128 (&fb)[TN]) {
#pragma unroll
    for (int i = 0; i < TM; ++i)
      fa[i] = *reinterpret_cast<const U128*>(&as[at(wr * (BM / 2) + i * 16 + fr, s * 4 + fk)]);
#pragma unroll
    for (int j = 0; j < TN; ++j)
      fb[j] = *reinterpret_cast<const U128*>(&bs[at(wc * (BN / 2) + j * 16 + fr, s * 4 + fk)]);
  };
  auto mma = [&](const U128 (&fa)[TM], const U128 (&fb)[TN]) {
#pragma unroll
    for (int i = 0; i < TM; ++i)
#pragma unroll
      for (int j = 0; j < TN; ++j)
        acc[i][j] = __builtin_amdgcn_mfma_f32_16x16x32_bf16(asBf16x8(fa[i]), asBf16x8(fb[j]),
                                                            acc[i][j], 0, 0, 0);
  };
  constexpr int kMm = TM * TN, kRd = TM + TN, kWr = AV + BV;
  static_assert(kMm >= kRd && (BK == 128 ? 2 * kMm >= kWr : kMm >= kWr),
                "MFMAs to interleave the memory instructions with");
  // A step whose stash and fetch both cover a whole slice: multiply (as, bs); write (xa, xb),
  // the next slice, into (na, nb); load slice k0f into (xa, xb) once written.
  auto wholeStep = [&](const uint16_t* as, const uint16_t* bs, U128 (&xa)[AV], U128 (&xb)[BV],
                       uint16_t* na, uint16_t* nb, int64_t k0f) {
    if constexpr (BK == 128) {
      // four 32-column sub-slices, fragments double-buffered in registers: each sub-slice's
      // reads go out during the MFMAs of the one before, the stash and the next loads during
      // the last two
      U128 fa[2][TM], fb[2][TN];
      frags(as, bs, 0, fa[0], fb[0]);
      frags(as, bs, 1, fa[1], fb[1]);
      mma(fa[0], fb[0]);
      frags(as, bs, 2, fa[0], fb[0]);
#pragma unroll
      for (int i = 0; i < kRd; ++i) {
        __builtin_amdgcn_sched_group_barrier(0x100, 1, 0);
        __builtin_amdgcn_sched_group_barrier(0x008, 1, 0);
      }
      mma(fa[1], fb[1]);
      frags(as, bs, 3, fa[1], fb[1]);
#pragma unroll
      for (int i = 0; i < kRd; ++i) {
        __builtin_amdgcn_sched_group_barrier(0x100, 1, 1);
        __builtin_amdgcn_sched_group_barrier(0x008, 1, 1);
      }
      stash(xa, xb, na, nb);
      fetchWhole(xa, xb, k0f);
      mma(fa[0], fb[0]);
      mma(fa[1], fb[1]);
#pragma unroll
      for (int i = 0; i < kWr / 2; ++i) {  // two LDS writes and two loads per MFMA
        __builtin_amdgcn_sched_group_barrier(0x200, 2, 2);
        __builtin_amdgcn_sched_group_barrier(0x008, 1, 2);
        __builtin_amdgcn_sched_group_barrier(0x020, 2, 2);
      }
      __syncthreads();
      return;
    }
    U128 fa0[TM], fb0[TN], fa1[TM], fb1[TN];
    frags(as, bs, 0, fa0, fb0);
    frags(as, bs, 1, fa1, fb1);
    mma(fa0, fb0);
#pragma unroll
    for (int i = 0; i < kRd; ++i) {
      __builtin_amdgcn_sched_group_barrier(0x100, 1, 0);  // one LDS read
      __builtin_amdgcn_sched_group_barrier(0x008, 2, 0);  // two MFMAs
    }
    if constexpr (kMm > kRd) __builtin_amdgcn_sched_group_barrier(0x008, kMm - kRd, 0);
    stash(xa, xb, na, nb);
    fetchWhole(xa, xb, k0f);
    mma(fa1, fb1);
#pragma unroll
    for (int i = 0; i < kWr; ++i) {
      __builtin_amdgcn_sched_group_barrier(0x200, 1, 1);  // one LDS write
      __builtin_amdgcn_sched_group_barrier(0x008, 2, 1);  // two MFMAs
      __builtin_amdgcn_sched_group_barrier(0x020, 1, 1);  // one global load
    }
    if constexpr (kMm > kWr) __builtin_amdgcn_sched_group_barrier(0x008, kMm - kWr, 1);
    __syncthreads();
  };
  // step s of nk near the end: stash and fetch only what exists
  auto tailStep = [&](const uint16_t* as, const uint16_t* bs, U128 (&xa)[AV], U128 (&xb)[BV],
                      uint16_t* na, uint16_t* nb, int64_t s, int64_t nk) {
    U128 fa[TM], fb[TN];
#pragma unroll
    for (int sub = 0; sub < BK / 32; ++sub) {
      frags(as, bs, sub, fa, fb);
      mma(fa, fb);
    }
    if (s + 1 < nk) stash(xa, xb, na, nb);
    __syncthreads();
    if (s + 3 < nk) fetch(xa, xb, (s + 3) * BK);
  };
  // slice j lives in registers j % 2 and LDS buffer j % 2
  U128 ra0[AV], rb0[BV], ra1[AV], rb1[BV];
  const int64_t nk = (K + BK - 1) / BK;
  fetch(ra0, rb0, 0);
  if (nk > 1) fetch(ra1, rb1, BK);
  stash(ra0, rb0, As0, Bs0);
  __syncthreads();
  if (nk > 2) fetch(ra0, rb0, 2 * BK);
  int64_t s = 0;
  for (; (s + 5) * BK <= K; s += 2) {  // steps s, s + 1 fetch slices s + 3, s + 4: all whole
    wholeStep(As0, Bs0, ra1, rb1, As1, Bs1, (s + 3) * BK);
    wholeStep(As1, Bs1, ra0, rb0, As0, Bs0, (s + 4) * BK);
  }
  for (; s < nk; s += 2) {
    tailStep(As0, Bs0, ra1, rb1, As1, Bs1, s, nk);
    if (s + 1 < nk) tailStep(As1, Bs1, ra0, rb0, As0, Bs0, s + 1, nk);
  }
  // Epilogue through LDS (every step ended with a barrier, so the operand buffers are free): the
  // accumulators go to LDS as fp32, then each thread takes runs of 8 consecutive columns of a
  // row, so bias / residual loads and output stores are 16-byte vectors. Runs that cross the
  // right edge, and outputs the vector forms cannot address, go element by element through the
  // same arithmetic.
  float* const ct = reinterpret_cast<float*>(smem);
#pragma unroll
  for (int i = 0; i < TM; ++i)
#pragma unroll
    for (int j = 0; j < TN; ++j)
#pragma unroll
      for (int v = 0; v < 4; ++v)
        ct[(wr * (BM / 2) + i * 16 + fk * 4 + v) * CP + wc * (BN / 2) + j * 16 + fr] =
            acc[i][j][v];
  __syncthreads();
  const bool vec = epi.vectorOk();
  if constexpr (Epi::kPairs) {
    // [gate 16 | up 16] column groups: run h (0, 1) of group b pairs gate columns 32 b + 8 h ..
    // with up columns 32 b + 16 + 8 h ..
    constexpr int kRuns = BM * BN / 16;
    static_assert(BN % 32 == 0 && kRuns % kGemmThreads == 0, "pair runs");
#pragma unroll
    for (int q = 0; q < kRuns / kGemmThreads; ++q) {
      const int e = t + q * kGemmThreads;
      const int row = e / (BN / 16), p = e % (BN / 16);
      const int cg = (p / 2) * 32 + (p % 2) * 8;
      const int64_t grow = r0 + row, gcol = c0 + cg;
      if (grow >= R) continue;
      float g[8], u[8];
#pragma unroll
      for (int k = 0; k < 8; ++k) {
        g[k] = ct[row * CP + cg + k];
        u[k] = ct[row * CP + cg + 16 + k];
      }
      if (vec && gcol + 24 <= Cn) {
        epi.pair8(grow, gcol, g, u);
      } else {
#pragma unroll
        for (int k = 0; k < 8; ++k)
          if (gcol + 16 + k < Cn) epi.pair(grow, gcol + k, g[k], u[k]);
      }
    }
  } else {
    // thread t's runs: rows t / (BN / 8) + q * (256 / (BN / 8)), all at column run c8. The
    // loads of every run go out before any result is stored: the compiler must assume a store
    // may alias a later run's input, so a load-compute-store loop per run waited for each load.
    constexpr int kRuns = BM * BN / 8, kPer = kRuns / kGemmThreads;
    static_assert(kRuns % kGemmThreads == 0 && kGemmThreads % (BN / 8) == 0, "runs");
    const int c8 = (t % (BN / 8)) * 8, row0 = t / (BN / 8);
    constexpr int kRowStep = kGemmThreads / (BN / 8);
    const int64_t gcol = c0 + c8;
    if (Epi::kVectorOnly || (vec && gcol + 8 <= Cn)) {
      const auto cd = epi.column(gcol);
      typename Epi::Run rd[kPer];
#pragma unroll
      for (int q = 0; q < kPer; ++q) {
        const int64_t grow = r0 + row0 + q * kRowStep;
        if (grow < R) rd[q] = epi.fetch(grow, gcol);
      }
#pragma unroll
      for (int q = 0; q < kPer; ++q) {
        const int row = row0 + q * kRowStep;
        const int64_t grow = r0 + row;
        if (grow >= R) continue;
        float v[8];
#pragma unroll
        for (int k = 0; k < 8; ++k) v[k] = ct[row * CP + c8 + k];
        epi.vec8(grow, gcol, v, cd, rd[q]);
      }
    } else if constexpr (!Epi::kVectorOnly) {
#pragma unroll
      for (int q = 0; q < kPer; ++q) {
        const int row = row0 + q * kRowStep;
        const int64_t grow = r0 + row;
        if (grow >= R) continue;
#pragma unroll
        for (int k = 0; k < 8; ++k)
          if (gcol + k < Cn) epi(grow, gcol + k, ct[row * CP + c8 + k]);
      }
    }
  }
}

// ---- epilogues ---------------------------------------------------------------------------------
// Scalar form epi(row, col, v) for any output; the bf16 GEMM also calls vec8(row, col, v[8]) (or
// pair8 for kPairs) for 8 consecutive columns when vectorOk(): the same arithmetic per element,
// with 16-byte loads and stores.

__device__ __forceinline__ bool aligned16(const void* p) {
  return (reinterpret_cast<uintptr_t>(p) & 15u) == 0;
}
// 8 bf16 of a 16-byte vector as floats
__device__ __forceinline__ void unpackBf16x8(const U128& w, float (&f)[8]) {
#pragma unroll
  for (int k = 0; k < 4; ++k) {
    f[2 * k] = __uint_as_float(w[k] << 16);
    f[2 * k + 1] = __uint_as_float(w[k] & 0xFFFF0000u);
  }
}
__device__ __forceinline__ U128 packBf16x8(const float (&f)[8]) {
  return U128{packBf16x2(f[0], f[1]), packBf16x2(f[2], f[3]), packBf16x2(f[4], f[5]),
              packBf16x2(f[6], f[7])};
}

// out[row * ldo + col] = act(v + bias[col]) as T
template <typename T, typename BiasT>
struct RowMajorOut {
  static constexpr bool kPairs = false;
  T* out;
  const BiasT* bias;
  int64_t ldo;
  int relu;
  __device__ __forceinline__ void operator()(int64_t row, int64_t col, float v) const {
    if (bias != nullptr) v += ld(bias + col);
    if (relu) v = fmaxf(v, 0.f);
    st(out + row * ldo + col, v);
  }
};

// RowMajorOut with the output type chosen at run time (one copy of the GEMM per kernel: two
// inlined copies, one per output type, took the kernel past 256 registers)
struct RowMajorOutBf16OrF32 {
  static constexpr bool kPairs = false;
  static constexpr bool kVectorOnly = false;
  void* out;
  const bf16* bias;
  int64_t ldo;
  int relu, out_f32;
  __device__ __forceinline__ void operator()(int64_t row, int64_t col, float v) const {
    if (bias != nullptr) v += ld(bias + col);
    if (relu) v = fmaxf(v, 0.f);
    if (out_f32)
      st(static_cast<float*>(out) + row * ldo + col, v);
    else
      st(static_cast<bf16*>(out) + row * ldo + col, v);
  }
  __device__ __forceinline__ bool vectorOk() const {
    return ldo % 8 == 0 && aligned16(out) && aligned16(bias);
  }
  struct Run {};
  __device__ __forceinline__ U128 column(int64_t col) const {
    return bias != nullptr ? gload16(bias + col) : zero16();
  }
  __device__ __forceinline__ Run fetch(int64_t, int64_t) const { return {}; }
  __device__ __forceinline__ void vec8(int64_t row, int64_t col, float (&v)[8], const U128& bw,
                                       const Run&) const {
    if (bias != nullptr) {
      float b[8];
      unpackBf16x8(bw, b);
#pragma unroll
      for (int k = 0; k < 8; ++k) v[k] += b[k];
    }
    if (relu)
#pragma unroll
      for (int k = 0; k < 8; ++k) v[k] = fmaxf(v[k], 0.f);
    if (out_f32) {
      float* o = static_cast<float*>(out) + row * ldo + col;
      *gp(reinterpret_cast<U128*>(o)) = U128{__float_as_uint(v[0]), __float_as_uint(v[1]),
                                             __float_as_uint(v[2]), __float_as_uint(v[3])};
      *gp(reinterpret_cast<U128*>(o + 4)) = U128{__float_as_uint(v[4]), __float_as_uint(v[5]),
                                                 __float_as_uint(v[6]), __float_as_uint(v[7])};
    } else {
      *gp(reinterpret_cast<U128*>(static_cast<bf16*>(out) + row * ldo + col)) = packBf16x8(v);
    }
  }
};

// out[row, col] = bf16(residual[row, col] + bf16(v + bias[col])): a linear whose output is
// added to the residual stream, rounded where the unfused graph rounds (linear, then add).
struct ResidualOut {
  static constexpr bool kPairs = false;
  static constexpr bool kVectorOnly = false;
  bf16* out;
  const bf16* residual;
  const bf16* bias;
  int64_t ldo;
  __device__ __forceinline__ void operator()(int64_t row, int64_t col, float v) const {
    if (bias != nullptr) v += ld(bias + col);
    const float o = Num<bf16>::round(v);
    st(out + row * ldo + col, ld(residual + row * ldo + col) + o);
  }
  __device__ __forceinline__ bool vectorOk() const {
    return ldo % 8 == 0 && aligned16(out) && aligned16(residual) && aligned16(bias);
  }
  using Run = U128;  // the residual run
  __device__ __forceinline__ U128 column(int64_t col) const {
    return bias != nullptr ? gload16(bias + col) : zero16();
  }
  __device__ __forceinline__ Run fetch(int64_t row, int64_t col) const {
    return gload16(residual + row * ldo + col);
  }
  __device__ __forceinline__ void vec8(int64_t row, int64_t col, float (&v)[8], const U128& bw,
                                       const Run& rw) const {
    if (bias != nullptr) {
      float b[8];
      unpackBf16x8(bw, b);
#pragma unroll
      for (int k = 0; k < 8; ++k) v[k] += b[k];
    }
    float r[8];
    unpackBf16x8(rw, r);
#pragma unroll
    for (int k = 0; k < 8; ++k) v[k] = r[k] + Num<bf16>::round(v[k]);
    *gp(reinterpret_cast<U128*>(out + row * ldo + col)) = packBf16x8(v);
  }
};

// SwiGLU of a [gate 16 | up 16]-interleaved weight (the layout of the fused decode weights):
// C columns 32 b + j (gate) and 32 b + 16 + j (up) give act[row, 16 b + j] =
// bf16(bf16(silu(bf16(gate))) * bf16(up)), the rounding points of the unfused linear, silu and
// mul nodes.
struct SwiGluOut {
  static constexpr bool kPairs = true;
  static constexpr bool kVectorOnly = false;
  bf16* out;
  int64_t ffn;
  __device__ __forceinline__ void pair(int64_t row, int64_t col, float gate, float up) const {
    FP_EXACT;
    const float g = Num<bf16>::round(gate), u = Num<bf16>::round(up);
    const float sg = Num<bf16>::round(g / (1.0f + expf(-g)));
    st(out + row * ffn + (col / 32) * 16 + col % 16, sg * u);
  }
  __device__ __forceinline__ bool vectorOk() const { return ffn % 8 == 0 && aligned16(out); }
  // gate columns col .. col + 7 (col % 16 == 0 or 8) with up columns col + 16 .. col + 23
  __device__ __forceinline__ void pair8(int64_t row, int64_t col, const float (&gate)[8],
                                        const float (&up)[8]) const {
    FP_EXACT;
    float o[8];
#pragma unroll
    for (int k = 0; k < 8; ++k) {
      const float g = Num<bf16>::round(gate[k]), u = Num<bf16>::round(up[k]);
      const float sg = Num<bf16>::round(g / (1.0f + expf(-g)));
      o[k] = sg * u;
    }
    *gp(reinterpret_cast<U128*>(out + row * ffn + (col / 32) * 16 + col % 16)) = packBf16x8(o);
  }
};

// The q|k|v projection of a prefill prompt straight into attention's layout: C row = token
// (b, s) of [B, S], C column = (q | k | v, head, d) of the packed [q; k; v] weight. Each value is
// rounded as the linear node rounds it (bf16(v + bias)); q and k then get the interleaved RoPE of
// position start_pos + s, rounded as the rotary node rounds it (pairs (2p, 2p + 1), positions
// outside the table copied unchanged); results go to q [B, Hq, S, D], k and v [B, Hkv, S, D]
// (rotary/kernel.py:6-35, and the reshape + transpose nodes a prompt needs). Vector form only:
// the host requires D % 8 == 0 and 16-byte aligned pointers (cos/sin too), so every 8-column
// run lies in one head and reads 16 bytes of each table row.
struct QkvHeadsOut {
  static constexpr bool kPairs = false;
  static constexpr bool kVectorOnly = true;
  bf16* q;
  bf16* k;
  bf16* v;
  const bf16* bias;
  const float* cosT;
  const float* sinT;
  int64_t seq, max_pos, start_pos;
  int q_heads, kv_heads, head_dim;
  __device__ __forceinline__ bool vectorOk() const { return true; }
  __device__ __forceinline__ void operator()(int64_t, int64_t, float) const {}
  // column-invariant part of a run: the bias and where the run goes
  struct Col {
    U128 bias;
    bf16* base;
    uint32_t heads, h, d;
  };
  struct Run {  // the table rows of the run's position
    U128 cs, sn;
  };
  __device__ __forceinline__ Col column(int64_t col) const {
    // 32-bit index arithmetic (the host bounds rows, columns and seq below 2^31)
    const uint32_t qw = static_cast<uint32_t>(q_heads * head_dim);
    const uint32_t kw = static_cast<uint32_t>(kv_heads * head_dim);
    const uint32_t cu = static_cast<uint32_t>(col);
    Col c;
    c.bias = gload16(bias + col);
    uint32_t rel;
    if (cu < qw) {
      c.base = q, rel = cu, c.heads = q_heads;
    } else if (cu < qw + kw) {
      c.base = k, rel = cu - qw, c.heads = kv_heads;
    } else {
      c.base = v, rel = cu - qw - kw, c.heads = kv_heads;
    }
    c.h = rel / static_cast<uint32_t>(head_dim);
    c.d = rel - c.h * static_cast<uint32_t>(head_dim);
    return c;
  }
  __device__ __forceinline__ int64_t position(int64_t row) const {
    return start_pos + static_cast<uint32_t>(row) % static_cast<uint32_t>(seq);
  }
  __device__ __forceinline__ Run fetch(int64_t row, int64_t col) const {
    // pairs d / 2 .. d / 2 + 3: 16 bytes of each table row (head_dim / 2 % 4 == 0); col is
    // recomputed into the head offset the way column() does
    const uint32_t hd = static_cast<uint32_t>(head_dim);
    const uint32_t qkw = static_cast<uint32_t>((q_heads + kv_heads) * head_dim);
    const int64_t pos = position(row);
    Run r{zero16(), zero16()};
    if (static_cast<uint32_t>(col) < qkw && pos >= 0 && pos < max_pos) {
      const int64_t at = pos * (head_dim / 2) + (static_cast<uint32_t>(col) % hd) / 2;
      r.cs = gload16(cosT + at);
      r.sn = gload16(sinT + at);
    }
    return r;
  }
  __device__ __forceinline__ void vec8(int64_t row, int64_t, float (&x)[8], const Col& c,
                                       const Run& r) const {
    FP_EXACT;
    float b8[8];
    unpackBf16x8(c.bias, b8);
#pragma unroll
    for (int e = 0; e < 8; ++e) x[e] = Num<bf16>::round(x[e] + b8[e]);
    const uint32_t ru = static_cast<uint32_t>(row), sq = static_cast<uint32_t>(seq);
    const uint32_t b = ru / sq, s = ru - b * sq;
    const int64_t pos = start_pos + s;
    if (c.base != v && pos >= 0 && pos < max_pos) {
#pragma unroll
      for (int j = 0; j < 4; ++j) {
        const float cs = __uint_as_float(r.cs[j]), sn = __uint_as_float(r.sn[j]);
        const float x0 = x[2 * j], x1 = x[2 * j + 1];
        x[2 * j] = x0 * cs - x1 * sn;
        x[2 * j + 1] = x0 * sn + x1 * cs;
      }
    }
    const uint64_t off =
        (static_cast<uint64_t>(b * c.heads + c.h) * sq + s) * static_cast<uint32_t>(head_dim) + c.d;
    *gp(reinterpret_cast<U128*>(c.base + off)) = packBf16x8(x);
  }
};

// out[n, oc, oy, ox] = act(v + bias[oc]) for C row oc and C column pixel (n, oy, ox)
struct ConvOut {
  static constexpr bool kPairs = false;
  float* out;
  const float* bias;
  int64_t OC, OHW;
  int relu;
  __device__ __forceinline__ void operator()(int64_t oc, int64_t pixel, float v) const {
    if (bias != nullptr) v += gp(bias)[oc];
    if (relu) v = fmaxf(v, 0.f);
    const int64_t n = pixel / OHW, p = pixel - n * OHW;
    gp(out)[(n * OC + oc) * OHW + p] = v;
  }
};

}  // namespace

// Tile sizes: _t64 for C up to a few hundred tiles of 64 x 64, _t128 for larger ones.
#define DK_MFMA_F32(BM, BN)                                                                     \
  extern "C" __global__ void __launch_bounds__(kGemmThreads)                                   \
      mfma_linear_f32_t##BM(const float* x, const float* w, const float* bias, float* out,     \
                            int64_t M, int64_t N, int64_t K, int relu) {                       \
    gemmF32<BM, BN>(RowsKT{{x, M, K, K}}, RowsKT{{w, N, K, K}}, M, N, K,                       \
                    RowMajorOut<float, float>{out, bias, N, relu});                            \
  }                                                                                            \
  extern "C" __global__ void __launch_bounds__(kGemmThreads)                                   \
      mfma_matmul_f32_t##BM(const float* a, const float* b, float* out, int64_t M, int64_t N,  \
                            int64_t K) {                                                       \
    gemmF32<BM, BN>(RowsKT{{a, M, K, K}}, KRowsT{{b, N, K, N}}, M, N, K,                       \
                    RowMajorOut<float, float>{out, nullptr, N, 0});                            \
  }                                                                                            \
  extern "C" __global__ void __launch_bounds__(kGemmThreads) mfma_conv2d_f32_t##BM(            \
      const float* x, const float* weight, const float* bias, float* out, int N, int C, int H, \
      int W, int OC, int KH, int KW, int OH, int OW, int SH, int SW, int PH, int PW, int relu) { \
    const int K = C * KH * KW, pixels = N * OH * OW;                                           \
    gemmF32<BM, BN>(RowsKT{{weight, OC, K, K}},                                                \
                    ConvPatch{x, pixels, K, 0, C, H, W, KH, KW, OH, OW, SH, SW, PH, PW}, OC,   \
                    pixels, K, ConvOut{out, bias, OC, static_cast<int64_t>(OH) * OW, relu});   \
  }

DK_MFMA_F32(64, 64)
DK_MFMA_F32(128, 128)

// Split-K conv2d for layers whose output tiles leave CUs with one workgroup: split z takes the
// patch elements [z * k_per_split, ...) and writes its partial [OC][pixels] tile to part[z];
// conv_splitk_reduce_f32 sums the splits in order, adds the bias, applies ReLU, writes NCHW.
extern "C" __global__ void __launch_bounds__(kGemmThreads) mfma_conv2d_f32_splitk_t64(
    const float* x, const float* weight, float* part, int N, int C, int H, int W, int OC, int KH,
    int KW, int OH, int OW, int SH, int SW, int PH, int PW, int k_per_split) {
  const int K = C * KH * KW, pixels = N * OH * OW;
  const int kb = static_cast<int>(blockIdx.z) * k_per_split;
  const int kl = K - kb < k_per_split ? K - kb : k_per_split;
  gemmF32<64, 64>(RowsKT{{weight + kb, OC, kl, K}},
                  ConvPatch{x, pixels, kl, kb, C, H, W, KH, KW, OH, OW, SH, SW, PH, PW}, OC,
                  pixels, kl,
                  RowMajorOut<float, float>{part + static_cast<int64_t>(blockIdx.z) * OC * pixels,
                                            nullptr, pixels, 0});
}

extern "C" __global__ void __launch_bounds__(kGemmThreads)
    conv_splitk_reduce_f32(const float* part, const float* bias, float* out, int64_t OC,
                           int64_t pixels, int64_t OHW, int splits, int relu) {
  const int64_t total = OC * pixels;
  for (int64_t e = static_cast<int64_t>(blockIdx.x) * kGemmThreads + threadIdx.x; e < total;
       e += static_cast<int64_t>(gridDim.x) * kGemmThreads) {
    float v = gp(part)[e];
    for (int z = 1; z < splits; ++z) v += gp(part)[z * total + e];
    const int64_t oc = e / pixels, pixel = e - oc * pixels;
    if (bias != nullptr) v += gp(bias)[oc];
    if (relu) v = fmaxf(v, 0.f);
    const int64_t n = pixel / OHW, q = pixel - n * OHW;
    gp(out)[(n * OC + oc) * OHW + q] = v;
  }
}

// Split-K fp32 linear for few output tiles and a long K (fully connected layers at small batch):
// split z = blockIdx.z takes k in [z * k_per_split, (z + 1) * k_per_split) and writes its
// partial tile to part[z][M][N]; splitk_reduce_f32 sums the splits in order (deterministic).
extern "C" __global__ void __launch_bounds__(kGemmThreads)
    mfma_linear_f32_splitk_t64(const float* x, const float* w, float* part, int64_t M, int64_t N,
                               int64_t K, int64_t k_per_split) {
  const int64_t kb = static_cast<int64_t>(blockIdx.z) * k_per_split;
  const int64_t kl = K - kb < k_per_split ? K - kb : k_per_split;
  gemmF32<64, 64>(RowsKT{{x + kb, M, kl, K}}, RowsKT{{w + kb, N, kl, K}}, M, N, kl,
                  RowMajorOut<float, float>{part + blockIdx.z * M * N, nullptr, N, 0});
}

extern "C" __global__ void __launch_bounds__(kGemmThreads)
    splitk_reduce_f32(const float* part, const float* bias, float* out, int64_t M, int64_t N,
                      int splits, int relu) {
  const int64_t total = M * N;
  for (int64_t e = static_cast<int64_t>(blockIdx.x) * kGemmThreads + threadIdx.x; e < total;
       e += static_cast<int64_t>(gridDim.x) * kGemmThreads) {
    float v = gp(part)[e];
    for (int z = 1; z < splits; ++z) v += gp(part)[z * total + e];
    if (bias != nullptr) v += gp(bias)[e % N];
    if (relu) v = fmaxf(v, 0.f);
    gp(out)[e] = v;
  }
}

// Two workgroups per CU (the LDS of two fits) and at most 256 VGPRs a lane: the compiler then
// keeps the accumulators in VGPRs and gives the two register stages and both sub-slices'
// fragments room without spilling.
#define DK_BF16_OCCUPANCY __attribute__((amdgpu_waves_per_eu(2)))

#define DK_MFMA_BF16(BM, BN)                                                                    \
  extern "C" __global__ void __launch_bounds__(kGemmThreads) DK_BF16_OCCUPANCY                   \
      mfma_linear_bf16_t##BM(                                                                  \
      const uint16_t* x, const uint16_t* w, const uint16_t* bias, void* out, int64_t M,        \
      int64_t N, int64_t K, int out_f32, int relu) {                                           \
    gemmBf16<BM, BN>(x, w, M, N, K, K,                                                         \
                     RowMajorOutBf16OrF32{out, reinterpret_cast<const bf16*>(bias), N, relu,   \
                                          out_f32});                                           \
  }

DK_MFMA_BF16(64, 64)
DK_MFMA_BF16(128, 128)

// bf16 linear + residual (bf16 out) and SwiGLU of an interleaved gate/up weight (N = 2 * ffn,
// ffn % 16 == 0): the ResidualOut and SwiGluOut epilogues above.
#define DK_MFMA_BF16_FUSED(BM, BN)                                                              \
  extern "C" __global__ void __launch_bounds__(kGemmThreads) DK_BF16_OCCUPANCY                   \
      mfma_linear_residual_bf16_t##BM(                                                         \
      const uint16_t* x, const uint16_t* w, const uint16_t* bias, const uint16_t* residual,    \
      uint16_t* out, int64_t M, int64_t N, int64_t K) {                                        \
    gemmBf16<BM, BN>(x, w, M, N, K, K,                                                         \
                     ResidualOut{reinterpret_cast<bf16*>(out),                                  \
                                 reinterpret_cast<const bf16*>(residual),                      \
                                 reinterpret_cast<const bf16*>(bias), N});                     \
  }                                                                                            \
  extern "C" __global__ void __launch_bounds__(kGemmThreads) DK_BF16_OCCUPANCY                   \
      mfma_gate_up_silu_bf16_t##BM(                                                            \
      const uint16_t* x, const uint16_t* w_gate_up, uint16_t* out, int64_t M, int64_t ffn,      \
      int64_t K) {                                                                             \
    gemmBf16<BM, BN>(x, w_gate_up, M, 2 * ffn, K, K,                                           \
                     SwiGluOut{reinterpret_cast<bf16*>(out), ffn});                             \
  }

DK_MFMA_BF16_FUSED(64, 64)
DK_MFMA_BF16_FUSED(128, 128)

// q|k|v projection + RoPE + head layout of a prefill prompt (QkvHeadsOut): x [B * S, K],
// w_qkv [(Hq + 2 Hkv) D, K], b_qkv [(Hq + 2 Hkv) D].
#define DK_MFMA_QKV_HEADS(BM, BN)                                                               \
  extern "C" __global__ void __launch_bounds__(kGemmThreads) DK_BF16_OCCUPANCY                 \
      mfma_qkv_heads_bf16_t##BM(const uint16_t* x, const uint16_t* w_qkv, const uint16_t* b_qkv, \
                                const float* cos, const float* sin, int64_t max_pos,           \
                                uint16_t* q, uint16_t* k, uint16_t* v, int64_t M, int64_t K,   \
                                int64_t seq, int64_t start_pos, int q_heads, int kv_heads,     \
                                int head_dim) {                                                \
    const int64_t n = static_cast<int64_t>(q_heads + 2 * kv_heads) * head_dim;                 \
    gemmBf16<BM, BN>(x, w_qkv, M, n, K, K,                                                     \
                     QkvHeadsOut{reinterpret_cast<bf16*>(q), reinterpret_cast<bf16*>(k),       \
                                 reinterpret_cast<bf16*>(v),                                   \
                                 reinterpret_cast<const bf16*>(b_qkv), cos, sin, seq, max_pos, \
                                 start_pos, q_heads, kv_heads, head_dim});                     \
  }

DK_MFMA_QKV_HEADS(64, 64)
DK_MFMA_QKV_HEADS(128, 128)

// bf16 linear with K split over grid.z (decode-sized m with few output tiles): part z covers
// columns [z * per, min(K, (z + 1) * per)) (per % 64 == 0) and writes its fp32 sums to
// part[z][M][N]; splitk_reduce_bf16 then adds the parts in z order.
extern "C" __global__ void __launch_bounds__(kGemmThreads) DK_BF16_OCCUPANCY
    mfma_linear_bf16_splitk_t64(const uint16_t* x, const uint16_t* w, float* part, int64_t M,
                                int64_t N, int64_t K, int64_t per) {
  const int64_t k0 = static_cast<int64_t>(blockIdx.z) * per;
  const int64_t len = K - k0 < per ? K - k0 : per;
  float* const out = part + static_cast<int64_t>(blockIdx.z) * M * N;
  gemmBf16<64, 64, 128, true>(x + k0, w + k0, M, N, len, K,
                              RowMajorOutBf16OrF32{out, nullptr, N, 0, 1});
}

// The same tile and slice shape without a split: decode-sized m (at most 64 rows), bias, bf16 or
// fp32 out; and with a residual (bf16 out).
extern "C" __global__ void __launch_bounds__(kGemmThreads) DK_BF16_OCCUPANCY
    mfma_linear_bf16_stream_t64(const uint16_t* x, const uint16_t* w, const uint16_t* bias,
                                void* out, int64_t M, int64_t N, int64_t K, int out_f32) {
  gemmBf16<64, 64, 128, true>(x, w, M, N, K, K,
                              RowMajorOutBf16OrF32{out, reinterpret_cast<const bf16*>(bias), N, 0,
                                                   out_f32});
}
extern "C" __global__ void __launch_bounds__(kGemmThreads) DK_BF16_OCCUPANCY
    mfma_linear_residual_bf16_stream_t64(const uint16_t* x, const uint16_t* w,
                                         const uint16_t* bias, const uint16_t* residual,
                                         uint16_t* out, int64_t M, int64_t N, int64_t K) {
  gemmBf16<64, 64, 128, true>(x, w, M, N, K, K,
                              ResidualOut{reinterpret_cast<bf16*>(out),
                                          reinterpret_cast<const bf16*>(residual),
                                          reinterpret_cast<const bf16*>(bias), N});
}

extern "C" __global__ void __launch_bounds__(kGemmThreads) DK_BF16_OCCUPANCY
    mfma_gate_up_silu_bf16_stream_t64(const uint16_t* x, const uint16_t* w_gate_up, uint16_t* out,
                                      int64_t M, int64_t ffn, int64_t K) {
  gemmBf16<64, 64, 128, true>(x, w_gate_up, M, 2 * ffn, K, K,
                              SwiGluOut{reinterpret_cast<bf16*>(out), ffn});
}

// out[m, n] = bf16(v + bias[n]), or with a residual bf16(residual[m, n] + bf16(v + bias[n])),
// v = the sum of the split parts in split order: the rounding points of RowMajorOut and
// ResidualOut.
extern "C" __global__ void __launch_bounds__(256)
    splitk_reduce_bf16(const float* part, const uint16_t* bias, const uint16_t* residual,
                       uint16_t* out, int64_t M, int64_t N, int splits) {
  const int64_t total = M * N;
  for (int64_t e = static_cast<int64_t>(blockIdx.x) * blockDim.x + threadIdx.x; e < total;
       e += static_cast<int64_t>(gridDim.x) * blockDim.x) {
    float v = gp(part)[e];
    for (int z = 1; z < splits; ++z) v += gp(part)[z * total + e];
    if (bias != nullptr) v += bf16ToFloat(gp(bias)[e % N]);
    if (residual != nullptr) v = bf16ToFloat(gp(residual)[e]) + Num<bf16>::round(v);
    gp(out)[e] = floatToBf16(v);
  }
}

// The split parts of the [q | k | v] projection of decode rows (one new token per row): each
// value is the sum of its parts in split order plus the bias, rounded to bf16 (the linear
// output); q and k columns are then rotated as interleaved pairs in fp32 and rounded again
// (rotary/kernel.py:6-35; no rotation at positions >= max_pos); q goes to q_out [M, Hq, D], k and
// v into the paged cache at the row's position (k_pool [block, Hkv, slot, D], v_pool [block, Hkv,
// D, slot]; rows whose position is negative or past the cache write nothing). The arithmetic is
// that of the qkv_rope_append decode kernels. One thread per (row, column pair): part reads and
// q / k stores are coalesced along the row.
extern "C" __global__ void __launch_bounds__(256)
    splitk_reduce_qkv_rope_append(const float* part, int splits, const uint16_t* bias,
                                  const float* cos_t, const float* sin_t, int64_t max_pos,
                                  const void* positions, int pos64, uint16_t* q_out,
                                  uint16_t* k_pool, uint16_t* v_pool, const int32_t* block_table,
                                  int64_t block_size, int64_t max_blocks, int M, int Hq, int Hkv,
                                  int D) {
  FP_EXACT;
  const int64_t N = static_cast<int64_t>(Hq + 2 * Hkv) * D;
  const int64_t pairs = N / 2;
  const int64_t total = static_cast<int64_t>(M) * pairs;
  const int64_t plane = static_cast<int64_t>(M) * N;
  const int64_t q_rows = static_cast<int64_t>(Hq) * D;
  const int64_t k_rows = static_cast<int64_t>(Hkv) * D;
  const int64_t capacity = max_blocks * block_size;
  for (int64_t e = static_cast<int64_t>(blockIdx.x) * blockDim.x + threadIdx.x; e < total;
       e += static_cast<int64_t>(gridDim.x) * blockDim.x) {
    const int m = static_cast<int>(e / pairs);
    const int64_t n = 2 * (e % pairs);
    const int64_t pos = loadIndex(positions, pos64, m);
    if (pos < 0) continue;
    const int64_t at = static_cast<int64_t>(m) * N + n;
    f32x2_t s = *gp(reinterpret_cast<const f32x2_t*>(part + at));
    for (int z = 1; z < splits; ++z) {
      const f32x2_t p = *gp(reinterpret_cast<const f32x2_t*>(part + z * plane + at));
      s.x += p.x;
      s.y += p.y;
    }
    if (bias != nullptr) {
      s.x += bf16ToFloat(gp(bias)[n]);
      s.y += bf16ToFloat(gp(bias)[n + 1]);
    }
    float v0 = Num<bf16>::round(s.x), v1 = Num<bf16>::round(s.y);
    const bool is_q = n < q_rows;
    const bool is_k = !is_q && n < q_rows + k_rows;
    const int64_t local = is_q ? n : (is_k ? n - q_rows : n - q_rows - k_rows);
    const int head = static_cast<int>(local / D);
    const int d = static_cast<int>(local % D);
    if ((is_q || is_k) && pos < max_pos) {
      const int64_t c = pos * (D / 2) + d / 2;
      const float cs = gp(cos_t)[c], sn = gp(sin_t)[c];
      const float r0 = v0 * cs - v1 * sn;
      const float r1 = v0 * sn + v1 * cs;
      v0 = r0;
      v1 = r1;
    }
    const uint32_t packed = packBf16x2(v0, v1);
    if (is_q) {
      *gp(reinterpret_cast<uint32_t*>(q_out + (static_cast<int64_t>(m) * Hq + head) * D + d)) =
          packed;
      continue;
    }
    if (pos >= capacity) continue;
    const int64_t blk = gp(block_table)[m * max_blocks + pos / block_size];
    const int64_t off = pos % block_size;
    if (is_k) {
      *gp(reinterpret_cast<uint32_t*>(k_pool + ((blk * Hkv + head) * block_size + off) * D + d)) =
          packed;
    } else {
      uint16_t* dst = v_pool + ((blk * Hkv + head) * D + d) * block_size + off;
      *gp(dst) = static_cast<uint16_t>(packed);
      *gp(dst + block_size) = static_cast<uint16_t>(packed >> 16);
    }
  }
}

// Split parts of a residual projection (o_proj, down_proj) of decode rows, then the RMSNorm that
// follows it: h = bf16(residual + bf16(sum of the parts in split order + bias)) (the values of
// splitk_reduce_bf16) and xn = bf16(h * rsqrt(mean(h^2) + eps) * norm_w)
// (rms_norm/kernel.py:6-14). One workgroup per row, h held in registers between the two; rows of
// N <= 4096 columns (N % 8 == 0), at most kMaxParts parts (2, 4 or 8: the kernel suffix). Every
// part of every chunk is requested before the first is added (the index of parts past `splits`
// is clamped and their sums discarded), so a row costs one memory round trip, not one per part,
// and the smallest kMaxParts that holds the parts keeps the surplus loads few.
constexpr int kResNormChunks = 2;
template <int kMaxParts>
__device__ __forceinline__ void splitkReduceResidualNorm(const float* part, int splits,
                                                         const uint16_t* bias,
                                                         const uint16_t* residual,
                                                         const uint16_t* norm_w, uint16_t* h_out,
                                                         uint16_t* xn_out, int M, int N,
                                                         float eps) {
  FP_EXACT;
  __shared__ float wave_sq[256 / kWave];
  const int m = blockIdx.x;
  const int chunks = N / 8;
  const int64_t plane = static_cast<int64_t>(M) * N;
  uint32_t h[kResNormChunks][4];
  float sq = 0.f;
#pragma unroll
  for (int c = 0; c < kResNormChunks; ++c) {
    const int i = threadIdx.x + c * 256;
    if (i >= chunks) break;
    const int64_t at = static_cast<int64_t>(m) * N + i * 8;
    f32x4 p[kMaxParts][2];
#pragma unroll
    for (int z = 0; z < kMaxParts; ++z) {
      const int64_t zz = z < splits ? z : splits - 1;
      p[z][0] = *gp(reinterpret_cast<const f32x4*>(part + zz * plane + at));
      p[z][1] = *gp(reinterpret_cast<const f32x4*>(part + zz * plane + at + 4));
    }
    const U128 r = gload16(residual + at);
    U128 b = U128{0u, 0u, 0u, 0u};
    if (bias != nullptr) b = gload16(bias + i * 8);
    float v[8];
#pragma unroll
    for (int e = 0; e < 8; ++e) v[e] = p[0][e / 4][e % 4];
#pragma unroll
    for (int z = 1; z < kMaxParts; ++z)
#pragma unroll
      for (int e = 0; e < 8; ++e) v[e] = z < splits ? v[e] + p[z][e / 4][e % 4] : v[e];
#pragma unroll
    for (int k = 0; k < 4; ++k) {
      float lo = v[2 * k], hi = v[2 * k + 1];
      if (bias != nullptr) {
        lo += __uint_as_float(b[k] << 16);
        hi += __uint_as_float(b[k] & 0xFFFF0000u);
      }
      lo = __uint_as_float(r[k] << 16) + Num<bf16>::round(lo);
      hi = __uint_as_float(r[k] & 0xFFFF0000u) + Num<bf16>::round(hi);
      h[c][k] = packBf16x2(lo, hi);
      const float hl = __uint_as_float(h[c][k] << 16), hh = __uint_as_float(h[c][k] & 0xFFFF0000u);
      sq += hl * hl;
      sq += hh * hh;
    }
    *gp(reinterpret_cast<U128*>(h_out + at)) = U128{h[c][0], h[c][1], h[c][2], h[c][3]};
  }
  sq = waveSum(sq);
  if (threadIdx.x % kWave == 0) wave_sq[threadIdx.x / kWave] = sq;
  __syncthreads();
  float total = 0.f;
#pragma unroll
  for (int w = 0; w < 256 / kWave; ++w) total += wave_sq[w];
  const float inv = 1.0f / sqrtf(total / static_cast<float>(N) + eps);
#pragma unroll
  for (int c = 0; c < kResNormChunks; ++c) {
    const int i = threadIdx.x + c * 256;
    if (i >= chunks) break;
    const U128 w = gload16(norm_w + i * 8);
    uint32_t o[4];
#pragma unroll
    for (int k = 0; k < 4; ++k) {
      const float hl = __uint_as_float(h[c][k] << 16), hh = __uint_as_float(h[c][k] & 0xFFFF0000u);
      o[k] = packBf16x2(hl * inv * __uint_as_float(w[k] << 16),
                        hh * inv * __uint_as_float(w[k] & 0xFFFF0000u));
    }
    *gp(reinterpret_cast<U128*>(xn_out + static_cast<int64_t>(m) * N + i * 8)) =
        U128{o[0], o[1], o[2], o[3]};
  }
}

#define DK_RESNORM(P)                                                                            \
  extern "C" __global__ void __launch_bounds__(256) splitk_reduce_residual_norm_p##P(           \
      const float* part, int splits, const uint16_t* bias, const uint16_t* residual,             \
      const uint16_t* norm_w, uint16_t* h_out, uint16_t* xn_out, int M, int N, float eps) {      \
    splitkReduceResidualNorm<P>(part, splits, bias, residual, norm_w, h_out, xn_out, M, N, eps); \
  }
DK_RESNORM(2)
DK_RESNORM(4)
DK_RESNORM(8)
