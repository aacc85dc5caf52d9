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

// bf16 rows with hidden % 8 == 0 and hidden <= 64 * 8 * kRowChunks (4096), 16-byte aligned: one wave
// per row (4 rows per 256-thread block, grid-stride over rows), the row held in registers as
// 16-byte chunks (chunk c of the row in lane c % 64), sum of squares reduced inside the wave
// (no LDS, no barrier), 16-byte loads and stores. Per element the same arithmetic as the
// block-per-row kernel: x * inv * w with inv = 1 / sqrt(mean(x^2) + eps), rounded once.
constexpr int kRowChunks = 8;

__device__ void rms_norm_rows_bf16(const uint16_t* x, const uint16_t* weight, uint16_t* out,
                                   int64_t rows, int hidden, float eps) {
  const int lane = threadIdx.x % kWave;
  const int chunks = hidden / 8;
  for (int64_t r = static_cast<int64_t>(blockIdx.x) * 4 + threadIdx.x / kWave; r < rows;
       r += static_cast<int64_t>(gridDim.x) * 4) {
    const uint16_t* row = x + r * hidden;
    uint32_t v[kRowChunks][4];
    float sq = 0.f;
#pragma unroll
    for (int c = 0; c < kRowChunks; ++c) {
      const int i = lane + c * kWave;
      if (i < chunks) {
        const uint4 w = *gp(reinterpret_cast<const uint4*>(row + i * 8));
        v[c][0] = w.x;
        v[c][1] = w.y;
        v[c][2] = w.z;
        v[c][3] = w.w;
#pragma unroll
        for (int k = 0; k < 4; ++k) {
          const float lo = __uint_as_float(v[c][k] << 16), hi = __uint_as_float(v[c][k] & 0xFFFF0000u);
          sq += lo * lo;
          sq += hi * hi;
        }
      }
    }
    const float inv = 1.0f / sqrtf(waveSum(sq) / static_cast<float>(hidden) + eps);
#pragma unroll
    for (int c = 0; c < kRowChunks; ++c) {
      const int i = lane + c * kWave;
      if (i < chunks) {
        const uint4 w = *gp(reinterpret_cast<const uint4*>(weight + i * 8));
        const uint32_t ww[4] = {w.x, w.y, w.z, w.w};
        uint32_t o[4];
#pragma unroll
        for (int k = 0; k < 4; ++k) {
          const float lo = __uint_as_float(v[c][k] << 16), hi = __uint_as_float(v[c][k] & 0xFFFF0000u);
          const float wlo = __uint_as_float(ww[k] << 16), whi = __uint_as_float(ww[k] & 0xFFFF0000u);
          o[k] = packBf16x2(lo * inv * wlo, hi * inv * whi);
        }
        *gp(reinterpret_cast<uint4*>(out + r * hidden + i * 8)) = uint4{o[0], o[1], o[2], o[3]};
      }
    }
  }
}

}  // namespace

extern "C" __global__ void __launch_bounds__(256)
    rms_norm_rows_bf16_k(const uint16_t* x, const uint16_t* weight, uint16_t* out, int64_t rows,
                         int hidden, float eps) {
  rms_norm_rows_bf16(x, weight, out, rows, hidden, eps);
}

DK_FLOAT_KERNELS(rms_norm, 256,
                 (const void* x, const void* weight, void* out, int64_t rows, int64_t hidden,
                  float eps),
                 (x, weight, out, rows, hidden, eps))
