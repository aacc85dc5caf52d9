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
//  mfma_linear_f32_splitk   fp32 linear with K split over grid.z into a workspace, then
//  + splitk_reduce_f32      a fixed-order sum with bias and ReLU
//
// Work split: a 256-thread workgroup owns a BM x BN tile of C (4 waves, 2 x 2, each BM/2 x BN/2
// as 16 x 16 MFMA tiles) and walks K in BK-wide slices. A slice of A and B is loaded from global
// memory into registers (coalesced: consecutive lanes take consecutive k of a row, or
// consecutive rows/pixels when those are contiguous in memory), written to LDS as [row][k] with
// a padded row pitch, and read back as MFMA fragments; the next slice's loads are in flight
// while the current one is multiplied. Rows, columns and k past the ends load zeros, so any
// shape works. Every output is a fixed-order sum: results do not depend on timing.
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

// Patch element k = (c, ky, kx) of output pixel `row` = (n, oy, ox) of a zero-padded NCHW conv.
// 32-bit index math (the host checks that every index fits).
struct ConvPatch {
  static constexpr bool kFastK = false;
  const float* x;
  int rows, K, C, H, W, KH, KW, OH, OW, SH, SW, PH, PW;
  __device__ __forceinline__ float load(int64_t row64, int64_t k64) const {
    const int row = static_cast<int>(row64), k = static_cast<int>(k64);
    if (row >= rows || k >= K) return 0.f;
    const int ox = row % OW, t = row / OW;
    const int oy = t % OH, n = t / OH;
    const int khw = KH * KW;
    const int c = k / khw, rem = k - c * khw;
    const int ky = rem / KW, kx = rem - ky * KW;
    const int iy = oy * SH + ky - PH, ix = ox * SW + kx - PW;
    if (iy < 0 || iy >= H || ix < 0 || ix >= W) return 0.f;
    return gp(x)[((n * C + c) * H + iy) * W + ix];
  }
};

// ---- fp32 core ---------------------------------------------------------------------------------
// v_mfma_f32_16x16x4_f32: lane l supplies A[l % 16][l / 16] and B[l / 16][l % 16] and receives
// D[(l / 16) * 4 + i][l % 16], i < 4.
template <int BM, int BN, class ASrc, class BSrc, class Epi>
__device__ __forceinline__ void gemmF32(const ASrc& A, const BSrc& B, int64_t R, int64_t Cn,
                                        int64_t K, const Epi& epi) {
  constexpr int BK = 32, LDK = BK + 4;  // pitch 36: the 16 rows x 4 k of a fragment read hit
                                        // 64 distinct banks
  constexpr int TM = BM / 32, TN = BN / 32;
  constexpr int AE = BM * BK / kGemmThreads, BE = BN * BK / kGemmThreads;
  __shared__ float As[BM * LDK];
  __shared__ float Bs[BN * LDK];
  const int t = threadIdx.x, lane = t % kWave, wave = t / kWave;
  const int wr = wave / 2, wc = wave % 2;
  const int64_t r0 = static_cast<int64_t>(blockIdx.y) * BM;
  const int64_t c0 = static_cast<int64_t>(blockIdx.x) * BN;
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
  auto fetch = [&](int64_t k0) {
#pragma unroll
    for (int i = 0; i < AE; ++i) {
      int row, k;
      slot(t + i * kGemmThreads, BM, ASrc::kFastK, row, k);
      ra[i] = A.load(r0 + row, k0 + k);
    }
#pragma unroll
    for (int i = 0; i < BE; ++i) {
      int row, k;
      slot(t + i * kGemmThreads, BN, BSrc::kFastK, row, k);
      rb[i] = B.load(c0 + row, k0 + k);
    }
  };
  auto stash = [&] {
#pragma unroll
    for (int i = 0; i < AE; ++i) {
      int row, k;
      slot(t + i * kGemmThreads, BM, ASrc::kFastK, row, k);
      As[row * LDK + k] = ra[i];
    }
#pragma unroll
    for (int i = 0; i < BE; ++i) {
      int row, k;
      slot(t + i * kGemmThreads, BN, BSrc::kFastK, row, k);
      Bs[row * LDK + k] = rb[i];
    }
  };
  f32x4 acc[TM][TN];
#pragma unroll
  for (int i = 0; i < TM; ++i)
#pragma unroll
    for (int j = 0; j < TN; ++j) acc[i][j] = f32x4{0.f, 0.f, 0.f, 0.f};
  const int fr = lane % 16, fk = lane / 16;
  fetch(0);
  for (int64_t k0 = 0; k0 < K; k0 += BK) {
    __syncthreads();  // every wave is done reading the previous slice
    stash();
    __syncthreads();
    if (k0 + BK < K) fetch(k0 + BK);
#pragma unroll
    for (int s = 0; s < BK / 4; ++s) {
      float a[TM], b[TN];
#pragma unroll
      for (int i = 0; i < TM; ++i) a[i] = As[(wr * (BM / 2) + i * 16 + fr) * LDK + s * 4 + fk];
#pragma unroll
      for (int j = 0; j < TN; ++j) b[j] = Bs[(wc * (BN / 2) + j * 16 + fr) * LDK + s * 4 + fk];
#pragma unroll
      for (int i = 0; i < TM; ++i)
#pragma unroll
        for (int j = 0; j < TN; ++j)
          acc[i][j] = __builtin_amdgcn_mfma_f32_16x16x4f32(a[i], b[j], acc[i][j], 0, 0, 0);
    }
  }
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

// ---- bf16 core ---------------------------------------------------------------------------------
// v_mfma_f32_16x16x32_bf16: lane l supplies A[l % 16][(l / 16) * 8 + j] and
// B[(l / 16) * 8 + j][l % 16], j < 8. Operands are [rows, K] row-major with K % 8 == 0 and
// 16-byte aligned rows, loaded 8 elements at a time.
template <int BM, int BN, class Epi>
__device__ __forceinline__ void gemmBf16(const uint16_t* a, const uint16_t* b, int64_t R,
                                         int64_t Cn, int64_t K, const Epi& epi) {
  constexpr int BK = 64, LDK = BK + 8;  // row pitch 144 bytes (16-byte aligned fragments)
  constexpr int TM = BM / 32, TN = BN / 32;
  constexpr int VPR = BK / 8;  // 16-byte vectors per tile row
  constexpr int AV = BM * VPR / kGemmThreads, BV = BN * VPR / kGemmThreads;
  __shared__ __attribute__((aligned(16))) uint16_t As[BM * LDK];
  __shared__ __attribute__((aligned(16))) uint16_t Bs[BN * LDK];
  const int t = threadIdx.x, lane = t % kWave, wave = t / kWave;
  const int wr = wave / 2, wc = wave % 2;
  const int64_t r0 = static_cast<int64_t>(blockIdx.y) * BM;
  const int64_t c0 = static_cast<int64_t>(blockIdx.x) * BN;
  U128 ra[AV], rb[BV];
  auto fetchOne = [&](const uint16_t* p, int64_t rows, int64_t row, int64_t k) {
    return row < rows && k < K ? gload16(p + row * K + k) : zero16();
  };
  auto fetch = [&](int64_t k0) {
#pragma unroll
    for (int i = 0; i < AV; ++i) {
      const int e = t + i * kGemmThreads;
      ra[i] = fetchOne(a, R, r0 + e / VPR, k0 + (e % VPR) * 8);
    }
#pragma unroll
    for (int i = 0; i < BV; ++i) {
      const int e = t + i * kGemmThreads;
      rb[i] = fetchOne(b, Cn, c0 + e / VPR, k0 + (e % VPR) * 8);
    }
  };
  auto stash = [&] {
#pragma unroll
    for (int i = 0; i < AV; ++i) {
      const int e = t + i * kGemmThreads;
      *reinterpret_cast<U128*>(&As[(e / VPR) * LDK + (e % VPR) * 8]) = ra[i];
    }
#pragma unroll
    for (int i = 0; i < BV; ++i) {
      const int e = t + i * kGemmThreads;
      *reinterpret_cast<U128*>(&Bs[(e / VPR) * LDK + (e % VPR) * 8]) = rb[i];
    }
  };
  f32x4 acc[TM][TN];
#pragma unroll
  for (int i = 0; i < TM; ++i)
#pragma unroll
    for (int j = 0; j < TN; ++j) acc[i][j] = f32x4{0.f, 0.f, 0.f, 0.f};
  const int fr = lane % 16, fk = lane / 16;
  fetch(0);
  for (int64_t k0 = 0; k0 < K; k0 += BK) {
    __syncthreads();
    stash();
    __syncthreads();
    if (k0 + BK < K) fetch(k0 + BK);
#pragma unroll
    for (int s = 0; s < BK / 32; ++s) {
      U128 fa[TM], fb[TN];
#pragma unroll
      for (int i = 0; i < TM; ++i)
        fa[i] = *reinterpret_cast<const U128*>(
            &As[(wr * (BM / 2) + i * 16 + fr) * LDK + s * 32 + fk * 8]);
#pragma unroll
      for (int j = 0; j < TN; ++j)
        fb[j] = *reinterpret_cast<const U128*>(
            &Bs[(wc * (BN / 2) + j * 16 + fr) * LDK + s * 32 + fk * 8]);
#pragma unroll
      for (int i = 0; i < TM; ++i)
#pragma unroll
        for (int j = 0; j < TN; ++j)
          acc[i][j] = __builtin_amdgcn_mfma_f32_16x16x32_bf16(asBf16x8(fa[i]), asBf16x8(fb[j]),
                                                              acc[i][j], 0, 0, 0);
    }
  }
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

// ---- epilogues ---------------------------------------------------------------------------------

// out[row * ldo + col] = act(v + bias[col]) as T
template <typename T, typename BiasT>
struct RowMajorOut {
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

// out[n, oc, oy, ox] = act(v + bias[oc]) for C row oc and C column pixel (n, oy, ox)
struct ConvOut {
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
    gemmF32<BM, BN>(RowsK{x, M, K, K}, RowsK{w, N, K, K}, M, N, K,                             \
                    RowMajorOut<float, float>{out, bias, N, relu});                            \
  }                                                                                            \
  extern "C" __global__ void __launch_bounds__(kGemmThreads)                                   \
      mfma_matmul_f32_t##BM(const float* a, const float* b, float* out, int64_t M, int64_t N,  \
                            int64_t K) {                                                       \
    gemmF32<BM, BN>(RowsK{a, M, K, K}, KRows{b, N, K, N}, M, N, K,                             \
                    RowMajorOut<float, float>{out, nullptr, N, 0});                            \
  }                                                                                            \
  extern "C" __global__ void __launch_bounds__(kGemmThreads) mfma_conv2d_f32_t##BM(            \
      const float* x, const float* weight, const float* bias, float* out, int N, int C, int H, \
      int W, int OC, int KH, int KW, int OH, int OW, int SH, int SW, int PH, int PW, int relu) { \
    const int K = C * KH * KW, pixels = N * OH * OW;                                           \
    gemmF32<BM, BN>(RowsK{weight, OC, K, K},                                                   \
                    ConvPatch{x, pixels, K, C, H, W, KH, KW, OH, OW, SH, SW, PH, PW}, OC,      \
                    pixels, K, ConvOut{out, bias, OC, static_cast<int64_t>(OH) * OW, relu});   \
  }

DK_MFMA_F32(64, 64)
DK_MFMA_F32(128, 128)

// Split-K fp32 linear for few output tiles and a long K (fully connected layers at small batch):
// split z = blockIdx.z takes k in [z * k_per_split, (z + 1) * k_per_split) and writes its
// partial tile to part[z][M][N]; splitk_reduce_f32 sums the splits in order (deterministic).
extern "C" __global__ void __launch_bounds__(kGemmThreads)
    mfma_linear_f32_splitk_t64(const float* x, const float* w, float* part, int64_t M, int64_t N,
                               int64_t K, int64_t k_per_split) {
  const int64_t kb = static_cast<int64_t>(blockIdx.z) * k_per_split;
  const int64_t kl = K - kb < k_per_split ? K - kb : k_per_split;
  gemmF32<64, 64>(RowsK{x + kb, M, kl, K}, RowsK{w + kb, N, kl, K}, M, N, kl,
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

#define DK_MFMA_BF16(BM, BN)                                                                    \
  extern "C" __global__ void __launch_bounds__(kGemmThreads) mfma_linear_bf16_t##BM(           \
      const uint16_t* x, const uint16_t* w, const uint16_t* bias, void* out, int64_t M,        \
      int64_t N, int64_t K, int out_f32, int relu) {                                           \
    const bf16* b = reinterpret_cast<const bf16*>(bias);                                       \
    if (out_f32)                                                                               \
      gemmBf16<BM, BN>(x, w, M, N, K,                                                          \
                       RowMajorOut<float, bf16>{static_cast<float*>(out), b, N, relu});        \
    else                                                                                       \
      gemmBf16<BM, BN>(x, w, M, N, K,                                                          \
                       RowMajorOut<bf16, bf16>{static_cast<bf16*>(out), b, N, relu});          \
  }

DK_MFMA_BF16(64, 64)
DK_MFMA_BF16(128, 128)
