// RMSNorm for gfx950: y = x * rsqrt(mean(x^2) + eps) * w (rms_norm/kernel.py:6-14).
// One 256-thread block per row; the row is read once into registers when it fits
// (hidden <= 256 * 8), else streamed twice. Sum of squares in fp32, block reduction through
// wave shuffles + LDS.
#include "common.h"

using namespace dk;

namespace {

template <typename T>
__device__ void rms_norm_impl(const void* x, const void* weight, void* out, int64_t rows,
                              int64_t hidden, float eps) {
  __shared__ float scratch[16];
  constexpr int kPer = 8;
  const T* px = static_cast<const T*>(x);
  const T* pw = static_cast<const T*>(weight);
  T* po = static_cast<T*>(out);
  const bool cached = hidden <= static_cast<int64_t>(blockDim.x) * kPer;
  for (int64_t r = blockIdx.x; r < rows; r += gridDim.x) {
    const T* row = px + r * hidden;
    float v[kPer];
    float sq = 0.f;
    if (cached) {
#pragma unroll
      for (int j = 0; j < kPer; ++j) {
        const int64_t i = threadIdx.x + static_cast<int64_t>(j) * blockDim.x;
        v[j] = i < hidden ? ld(row + i) : 0.f;
        sq += v[j] * v[j];
      }
    } else {
      for (int64_t i = threadIdx.x; i < hidden; i += blockDim.x) {
        const float e = ld(row + i);
        sq += e * e;
      }
    }
    const float inv = 1.0f / sqrtf(blockSum(sq, scratch) / static_cast<float>(hidden) + eps);
    if (cached) {
#pragma unroll
      for (int j = 0; j < kPer; ++j) {
        const int64_t i = threadIdx.x + static_cast<int64_t>(j) * blockDim.x;
        if (i < hidden) st(po + r * hidden + i, v[j] * inv * ld(pw + i));
      }
    } else {
      for (int64_t i = threadIdx.x; i < hidden; i += blockDim.x)
        st(po + r * hidden + i, ld(row + i) * inv * ld(pw + i));
    }
  }
}

}  // namespace

DK_FLOAT_KERNELS(rms_norm, 256,
                 (const void* x, const void* weight, void* out, int64_t rows, int64_t hidden,
                  float eps),
                 (x, weight, out, rows, hidden, eps))
