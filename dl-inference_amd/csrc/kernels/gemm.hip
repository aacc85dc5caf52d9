// GEMM kernels for the `linear` and `matmul` operators on gfx950.
//
//  gemm_tiled_<t>   any dtype/shape: 64x64 output tile per 256-thread block, k in steps of 16
//                   through LDS, 4x4 outputs per thread, fp32 accumulation.
//                   linear/kernel.py:6-44 (w is [n, k]) and matmul/kernel.py:6-40 (b is [k, n]).
//  skinny_linear_<MB>  bf16 weight streaming for m <= 16 * MB rows (decode): MFMA core from
//                   skinny.h, bias epilogue, bf16 or fp32 output.
#include "common.h"
#include "skinny.h"

using namespace dk;

namespace {

template <typename T>
__device__ void gemm_tiled_impl(const void* a_, const void* b_, const void* bias_, void* out_,
                                int64_t M, int64_t N, int64_t K, int b_is_nk, int out_f32) {
  constexpr int BM = 64, BN = 64, BK = 16;
  __shared__ float As[BK][BM + 4];
  __shared__ float Bs[BK][BN + 4];
  const T* A = static_cast<const T*>(a_);
  const T* B = static_cast<const T*>(b_);
  const int t = threadIdx.x;
  const int64_t m0 = static_cast<int64_t>(blockIdx.y) * BM;
  const int64_t n0 = static_cast<int64_t>(blockIdx.x) * BN;
  const int ty = t / 16, tx = t % 16;
  float acc[4][4] = {};

  for (int64_t k0 = 0; k0 < K; k0 += BK) {
    // A tile: 64 rows x 16 k; thread -> row t/4, k (t%4)*4 .. +3
    {
      const int row = t / 4, kk = (t % 4) * 4;
      const int64_t m = m0 + row;
#pragma unroll
      for (int j = 0; j < 4; ++j) {
        const int64_t k = k0 + kk + j;
        As[kk + j][row] = (m < M && k < K) ? ld(A + m * K + k) : 0.f;
      }
    }
    if (b_is_nk) {  // B given as [N, K]
      const int col = t / 4, kk = (t % 4) * 4;
      const int64_t n = n0 + col;
#pragma unroll
      for (int j = 0; j < 4; ++j) {
        const int64_t k = k0 + kk + j;
        Bs[kk + j][col] = (n < N && k < K) ? ld(B + n * K + k) : 0.f;
      }
    } else {  // B given as [K, N]
      const int kk = t / 16, col = (t % 16) * 4;
      const int64_t k = k0 + kk;
#pragma unroll
      for (int j = 0; j < 4; ++j) {
        const int64_t n = n0 + col + j;
        Bs[kk][col + j] = (n < N && k < K) ? ld(B + k * N + n) : 0.f;
      }
    }
    __syncthreads();
#pragma unroll
    for (int kk = 0; kk < BK; ++kk) {
      float av[4], bv[4];
#pragma unroll
      for (int i = 0; i < 4; ++i) av[i] = As[kk][ty * 4 + i];
#pragma unroll
      for (int j = 0; j < 4; ++j) bv[j] = Bs[kk][tx * 4 + j];
#pragma unroll
      for (int i = 0; i < 4; ++i)
#pragma unroll
        for (int j = 0; j < 4; ++j) acc[i][j] = fmaf(av[i], bv[j], acc[i][j]);
    }
    __syncthreads();
  }

#pragma unroll
  for (int i = 0; i < 4; ++i) {
    const int64_t m = m0 + ty * 4 + i;
    if (m >= M) continue;
#pragma unroll
    for (int j = 0; j < 4; ++j) {
      const int64_t n = n0 + tx * 4 + j;
      if (n >= N) continue;
      float v = acc[i][j];
      if (bias_ != nullptr) v += ld(static_cast<const T*>(bias_) + n);
      if (out_f32)
        static_cast<float*>(out_)[m * N + n] = v;
      else
        st(static_cast<T*>(out_) + m * N + n, v);
    }
  }
}

// Skinny linear: grid (ceil(N / 32), 1), 256 threads. Requires K % 64 == 0 and 16-byte aligned
// rows (checked on the host).
template <int MB>
__device__ void skinny_linear_impl(const uint16_t* x, const uint16_t* w, const uint16_t* bias,
                                   void* out, int64_t M, int64_t N, int64_t K, int out_f32) {
  using Core = SkinnyCore<2, MB, 4>;
  __shared__ float lds[Core::kLdsFloats];
  const int64_t n0 = static_cast<int64_t>(blockIdx.x) * Core::kTileN;
  Core::run(w, XGlobal{x, K}, N, K, static_cast<int>(M), n0, 0, static_cast<int>(K / 64), lds);
  for (int idx = threadIdx.x; idx < Core::kTileN * Core::kTileM; idx += 4 * kWave) {
    const int nl = idx / Core::kTileM, m = idx % Core::kTileM;
    const int64_t n = n0 + nl;
    if (m >= M || n >= N) continue;
    float v = lds[idx];
    if (bias != nullptr) v += bf16ToFloat(bias[n]);
    if (out_f32)
      static_cast<float*>(out)[m * N + n] = v;
    else
      static_cast<uint16_t*>(out)[m * N + n] = floatToBf16(v);
  }
}

}  // namespace

DK_FLOAT_KERNELS(gemm_tiled, 256,
                 (const void* a, const void* b, const void* bias, void* out, int64_t M, int64_t N,
                  int64_t K, int b_is_nk, int out_f32),
                 (a, b, bias, out, M, N, K, b_is_nk, out_f32))

#define DK_SKINNY_LINEAR(MB)                                                                \
  extern "C" __global__ void __launch_bounds__(256)                                         \
      skinny_linear_m##MB(const uint16_t* x, const uint16_t* w, const uint16_t* bias,       \
                          void* out, int64_t M, int64_t N, int64_t K, int out_f32) {        \
    skinny_linear_impl<MB>(x, w, bias, out, M, N, K, out_f32);                              \
  }
DK_SKINNY_LINEAR(1)
DK_SKINNY_LINEAR(2)
DK_SKINNY_LINEAR(4)
