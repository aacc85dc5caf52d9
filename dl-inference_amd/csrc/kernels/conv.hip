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

// ---------------------------------------------------------------------------------------------
// fp32 convolution with a small patch (in_c * kh * kw of 9 or 27), e.g. an RGB input layer:
// as a GEMM its reduction is too short for MFMA tiles to pay (27 for 3 x 3 x 3), and the layer is
// bound by writing its output. Thread = one output pixel (n, oy, ox) for kSmallOc consecutive
// output channels (grid.y over channel groups): it gathers the pixel's patch into registers
// (zero outside the image; the patch element -> (input offset, ky, kx) table comes in the kernel
// arguments), then sums bias + patch . filter in (c, ky, kx) order per channel, applies ReLU if
// asked and stores NCHW, consecutive threads writing consecutive ox. Table and filters are the
// same for every lane, so both reach the lanes through scalar loads, not LDS (whose bandwidth a
// per-lane copy of every filter element would exhaust).
// ---------------------------------------------------------------------------------------------
#include "conv_small.h"

namespace {

// kP: the patch size C * KH * KW (a compile-time constant, so that each filter arrives in whole
// s_load_dwordx16 batches and the loops carry no bounds checks).
template <int kP>
__device__ void convSmall(const float* __restrict__ x, const float* __restrict__ w,
                          const float* __restrict__ bias, float* __restrict__ out, int N, int C,
                          int H, int W, int OC, int OH, int OW, int SH, int SW, int PH, int PW,
                          int relu, const dk::SmallConvTable& tab) {
  using dk::kSmallOc;
  static_assert(kP <= dk::kSmallPatch, "table size");
  constexpr int patch = kP;
  const int oc0 = blockIdx.y * kSmallOc;
  // 32-bit index math: the host keeps every pixel and element index below 2^31
  const unsigned pixels = static_cast<unsigned>(N) * OH * OW;
  const unsigned p = blockIdx.x * blockDim.x + threadIdx.x;
  if (p >= pixels) return;
  const unsigned row = p / static_cast<unsigned>(OW);
  const int ox = static_cast<int>(p - row * OW);
  const unsigned img = row / static_cast<unsigned>(OH);
  const int oy = static_cast<int>(row - img * OH);
  const int n = static_cast<int>(img);
  const int iy0 = oy * SH - PH, ix0 = ox * SW - PW;
  const float* const xb =
      x + static_cast<int64_t>(n) * C * H * W + static_cast<int64_t>(iy0) * W + ix0;
  float v[kP];
#pragma unroll
  for (int k = 0; k < kP; ++k) {
    const int iy = iy0 + tab.ky[k], ix = ix0 + tab.kx[k];
    v[k] = iy >= 0 && iy < H && ix >= 0 && ix < W ? xb[tab.offset[k]] : 0.f;
  }
  const int64_t plane = static_cast<int64_t>(OH) * OW;
  float* const o = out + static_cast<int64_t>(n) * OC * plane + static_cast<int64_t>(oy) * OW + ox;
  const float* const filters = w + static_cast<int64_t>(oc0) * patch;
#pragma unroll
  for (int j = 0; j < kSmallOc; ++j) {
    if (oc0 + j >= OC) break;
    const float* const f = filters + j * patch;
    float acc = bias != nullptr ? bias[oc0 + j] : 0.f;
#pragma unroll
    for (int k = 0; k < kP; ++k) acc = fmaf(v[k], f[k], acc);
    if (relu && acc < 0.f) acc = 0.f;
    o[static_cast<int64_t>(oc0 + j) * plane] = acc;
  }
}

}  // namespace

#define DK_CONV_SMALL(P)                                                                        \
  extern "C" __global__ void __launch_bounds__(256) conv2d_small_f32_p##P(                     \
      const float* __restrict__ x, const float* __restrict__ w, const float* __restrict__ bias, \
      float* __restrict__ out, int N, int C, int H, int W, int OC, int OH, int OW, int SH,      \
      int SW, int PH, int PW, int relu, dk::SmallConvTable tab) {                               \
    convSmall<P>(x, w, bias, out, N, C, H, W, OC, OH, OW, SH, SW, PH, PW, relu, tab);          \
  }

DK_CONV_SMALL(9)   // one channel, 3 x 3
DK_CONV_SMALL(27)  // three channels (RGB), 3 x 3
