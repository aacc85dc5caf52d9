// Direct NCHW convolution (conv2d/kernel.py:6-49): one thread per output element, zero
// padding, optional bias, fp32 accumulation. Weights of one output channel are reused from
// L1/L2 across the threads of a block because consecutive threads share (n, oc) and differ in
// the output pixel.
#include "common.h"

using namespace dk;

namespace {

template <typename T>
__device__ void conv2d_impl(const void* x_, const void* w_, const void* bias_, void* out_,
                            int64_t N, int64_t C, int64_t H, int64_t W, int64_t OC, int64_t KH,
                            int64_t KW, int64_t OH, int64_t OW, int64_t SH, int64_t SW,
                            int64_t PH, int64_t PW) {
  const T* x = static_cast<const T*>(x_);
  const T* w = static_cast<const T*>(w_);
  T* out = static_cast<T*>(out_);
  const int64_t total = N * OC * OH * OW;
  for (int64_t e = static_cast<int64_t>(blockIdx.x) * blockDim.x + threadIdx.x; e < total;
       e += static_cast<int64_t>(gridDim.x) * blockDim.x) {
    const int64_t ox = e % OW;
    const int64_t oy = (e / OW) % OH;
    const int64_t oc = (e / (OW * OH)) % OC;
    const int64_t n = e / (OW * OH * OC);
    float acc = bias_ != nullptr ? ld(static_cast<const T*>(bias_) + oc) : 0.f;
    for (int64_t c = 0; c < C; ++c) {
      const T* plane = x + (n * C + c) * H * W;
      const T* filt = w + (oc * C + c) * KH * KW;
      for (int64_t ky = 0; ky < KH; ++ky) {
        const int64_t iy = oy * SH + ky - PH;
        if (iy < 0 || iy >= H) continue;
        for (int64_t kx = 0; kx < KW; ++kx) {
          const int64_t ix = ox * SW + kx - PW;
          if (ix < 0 || ix >= W) continue;
          acc = fmaf(ld(plane + iy * W + ix), ld(filt + ky * KW + kx), acc);
        }
      }
    }
    st(out + e, acc);
  }
}

}  // namespace

DK_FLOAT_KERNELS(conv2d, 256,
                 (const void* x, const void* w, const void* bias, void* out, int64_t N, int64_t C,
                  int64_t H, int64_t W, int64_t OC, int64_t KH, int64_t KW, int64_t OH, int64_t OW,
                  int64_t SH, int64_t SW, int64_t PH, int64_t PW),
                 (x, w, bias, out, N, C, H, W, OC, KH, KW, OH, OW, SH, SW, PH, PW))
