// Elementwise, gather, reduction-per-row and layout kernels for gfx950.
// Semantics follow the reference Triton kernels cited per kernel; all math in fp32.
#include "common.h"

using namespace dk;

namespace {

// Grid-stride over `total` elements; 256 threads, each handling 4 consecutive-stride items.
#define DK_GRID_STRIDE(i, total)                                                   \
  for (int64_t i = static_cast<int64_t>(blockIdx.x) * blockDim.x + threadIdx.x; i < (total); \
       i += static_cast<int64_t>(gridDim.x) * blockDim.x)

// add/kernel.py:6-11 — out[i] = a[i] + b[i % width]
template <typename T>
__device__ void add_impl(const void* a, const void* b, void* out, int64_t total, int64_t width) {
  const T* pa = static_cast<const T*>(a);
  const T* pb = static_cast<const T*>(b);
  T* po = static_cast<T*>(out);
  DK_GRID_STRIDE(i, total) { st(po + i, ld(pa + i) + ld(pb + i % width)); }
}

// mul/kernel.py:6-11 — out[i] = a[i] * b[i % width]
template <typename T>
__device__ void mul_impl(const void* a, const void* b, void* out, int64_t total, int64_t width) {
  const T* pa = static_cast<const T*>(a);
  const T* pb = static_cast<const T*>(b);
  T* po = static_cast<T*>(out);
  DK_GRID_STRIDE(i, total) { st(po + i, ld(pa + i) * ld(pb + i % width)); }
}

// silu/kernel.py:6-10 — x / (1 + exp(-x))
template <typename T>
__device__ void silu_impl(const void* x, void* out, int64_t total) {
  const T* px = static_cast<const T*>(x);
  T* po = static_cast<T*>(out);
  DK_GRID_STRIDE(i, total) {
    const float v = ld(px + i);
    st(po + i, v / (1.0f + __expf(-v)));
  }
}

// relu/kernel.py:6-10 — max(x, 0)
template <typename T>
__device__ void relu_impl(const void* x, void* out, int64_t total) {
  const T* px = static_cast<const T*>(x);
  T* po = static_cast<T*>(out);
  DK_GRID_STRIDE(i, total) { st(po + i, fmaxf(ld(px + i), 0.0f)); }
}

// batch_norm2d/kernel.py:6-28 — (x - mean) * rsqrt(var + eps) * w + b, channel = (i / spatial) % C
template <typename T>
__device__ void batch_norm2d_impl(const void* x, const void* w, const void* b, const void* mean,
                                  const void* var, void* out, int64_t total, int64_t channels,
                                  int64_t spatial, float eps) {
  const T* px = static_cast<const T*>(x);
  T* po = static_cast<T*>(out);
  DK_GRID_STRIDE(i, total) {
    const int64_t c = (i / spatial) % channels;
    const float inv = rsqrtf(ld(static_cast<const T*>(var) + c) + eps);
    const float norm = (ld(px + i) - ld(static_cast<const T*>(mean) + c)) * inv;
    st(po + i, norm * ld(static_cast<const T*>(w) + c) + ld(static_cast<const T*>(b) + c));
  }
}

// max_pool2d/kernel.py:6-41 — window max, padding contributes -inf
template <typename T>
__device__ void max_pool2d_impl(const void* x, void* out, int64_t n, int64_t c, int64_t h,
                                int64_t w, int64_t oh, int64_t ow, int64_t kh, int64_t kw,
                                int64_t sh, int64_t sw, int64_t ph, int64_t pw) {
  const T* px = static_cast<const T*>(x);
  T* po = static_cast<T*>(out);
  const int64_t total = n * c * oh * ow;
  DK_GRID_STRIDE(i, total) {
    const int64_t ox = i % ow;
    const int64_t oy = (i / ow) % oh;
    const int64_t plane = i / (ow * oh);  // n * c + channel
    float best = -INFINITY;
    for (int64_t dy = 0; dy < kh; ++dy) {
      const int64_t iy = oy * sh + dy - ph;
      if (iy < 0 || iy >= h) continue;
      for (int64_t dx = 0; dx < kw; ++dx) {
        const int64_t ix = ox * sw + dx - pw;
        if (ix < 0 || ix >= w) continue;
        best = fmaxf(best, ld(px + (plane * h + iy) * w + ix));
      }
    }
    st(po + i, best);
  }
}

// embedding/kernel.py:6-23 — one block per token row; out-of-range ids give a zero row.
template <typename T>
__device__ void embedding_impl(const void* ids, int ids64, const void* table, void* out,
                               int64_t tokens, int64_t hidden, int64_t vocab) {
  const T* pt = static_cast<const T*>(table);
  T* po = static_cast<T*>(out);
  for (int64_t t = blockIdx.x; t < tokens; t += gridDim.x) {
    const int64_t id = loadIndex(ids, ids64, t);
    const bool valid = id >= 0 && id < vocab;
    for (int64_t d = threadIdx.x; d < hidden; d += blockDim.x)
      po[t * hidden + d] = valid ? pt[id * hidden + d] : T{};
  }
}

// softmax/kernel.py:6-14 — one block per row, any width (three passes over the row).
template <typename T>
__device__ void softmax_impl(const void* x, void* out, int64_t rows, int64_t width) {
  __shared__ float scratch[16];
  const T* px = static_cast<const T*>(x);
  T* po = static_cast<T*>(out);
  for (int64_t r = blockIdx.x; r < rows; r += gridDim.x) {
    const T* row = px + r * width;
    float m = -INFINITY;
    for (int64_t i = threadIdx.x; i < width; i += blockDim.x) m = fmaxf(m, ld(row + i));
    m = blockMax(m, scratch);
    float s = 0.f;
    for (int64_t i = threadIdx.x; i < width; i += blockDim.x) s += __expf(ld(row + i) - m);
    s = blockSum(s, scratch);
    const float inv = 1.0f / s;
    for (int64_t i = threadIdx.x; i < width; i += blockDim.x)
      st(po + r * width + i, __expf(ld(row + i) - m) * inv);
  }
}

// transpose/kernel.py:6-20 — 32x32 tiles through LDS, +1 column of padding against bank clashes.
template <typename T>
__device__ void transpose2d_impl(const void* x, void* out, int64_t rows, int64_t cols) {
  __shared__ float tile[32][33];
  const T* px = static_cast<const T*>(x);
  T* po = static_cast<T*>(out);
  const int64_t r0 = static_cast<int64_t>(blockIdx.y) * 32;
  const int64_t c0 = static_cast<int64_t>(blockIdx.x) * 32;
  const int tx = threadIdx.x % 32;
  const int ty = threadIdx.x / 32;  // 0..7
  for (int k = ty; k < 32; k += 8) {
    const int64_t r = r0 + k, c = c0 + tx;
    tile[k][tx] = (r < rows && c < cols) ? ld(px + r * cols + c) : 0.f;
  }
  __syncthreads();
  for (int k = ty; k < 32; k += 8) {
    const int64_t c = c0 + k, r = r0 + tx;
    if (r < rows && c < cols) st(po + c * rows + r, tile[tx][k]);
  }
}

// out[a, c, b, :] = x[a, b, c, :] for x [n0, n1, n2, row] (permutation [0, 2, 1, 3]): the
// [B, S, H, D] <-> [B, H, S, D] change of a prefill graph, which the reference's 2-D transpose
// (transpose/kernel.py:6-20) cannot express. Rows of `row` units (16 bytes each when the row
// bytes allow, else 2 bytes) are copied whole, so reads and writes stay contiguous per row.
template <typename U>
__device__ void permute_0213_impl(const void* x, void* out, int64_t n0, int64_t n1, int64_t n2,
                                  int64_t row) {
  const U* px = static_cast<const U*>(x);
  U* po = static_cast<U*>(out);
  const int64_t total = n0 * n1 * n2 * row;
  DK_GRID_STRIDE(i, total) {
    const int64_t e = i % row;
    int64_t r = i / row;  // output row (a, c, b)
    const int64_t b = r % n1;
    r /= n1;
    const int64_t c = r % n2;
    const int64_t a = r / n2;
    po[i] = px[((a * n1 + b) * n2 + c) * row + e];
  }
}

// rotary/kernel.py:6-35 — interleaved pairs (2p, 2p+1). One thread per (vector, pair) for q,
// then for k. Pairs beyond `pairs` (dims >= 2*pairs) are copied unchanged.
template <typename T>
__device__ void rotate_tensor(const T* x, T* out, int64_t vectors, int64_t heads, int64_t seq,
                              int64_t head_dim, int64_t pairs, const float* cosT, const float* sinT,
                              int64_t max_pos, int64_t start_pos, const void* positions, int pos64) {
  const int64_t half = head_dim / 2;
  const int64_t work = vectors * half;
  DK_GRID_STRIDE(i, work) {
    const int64_t p = i % half;
    const int64_t vec = i / half;  // ((b * heads + h) * seq + t)
    const int64_t t = vec % seq;
    const int64_t b = vec / (seq * heads);
    int64_t pos = start_pos + t;
    if (positions != nullptr) pos += loadIndex(positions, pos64, b);
    const int64_t base = vec * head_dim + 2 * p;
    const float x0 = ld(x + base);
    const float x1 = ld(x + base + 1);
    if (p < pairs && pos >= 0 && pos < max_pos) {
      const float c = cosT[pos * pairs + p];
      const float s = sinT[pos * pairs + p];
      st(out + base, x0 * c - x1 * s);
      st(out + base + 1, x0 * s + x1 * c);
    } else {
      st(out + base, x0);
      st(out + base + 1, x1);
    }
  }
}

template <typename T>
__device__ void rotary_impl(const void* q, const void* k, const float* cosT, const float* sinT,
                            void* out_q, void* out_k, int64_t batch, int64_t q_heads,
                            int64_t k_heads, int64_t seq, int64_t head_dim, int64_t pairs,
                            int64_t max_pos, int64_t start_pos, const void* positions, int pos64) {
  rotate_tensor(static_cast<const T*>(q), static_cast<T*>(out_q), batch * q_heads * seq, q_heads,
                seq, head_dim, pairs, cosT, sinT, max_pos, start_pos, positions, pos64);
  rotate_tensor(static_cast<const T*>(k), static_cast<T*>(out_k), batch * k_heads * seq, k_heads,
                seq, head_dim, pairs, cosT, sinT, max_pos, start_pos, positions, pos64);
}

// torch.argmax rule: the first index of the maximum. One block per row.
template <typename T>
__device__ void argmax_impl(const void* x, int64_t* ids, int64_t rows, int64_t width) {
  __shared__ float best_v[16];
  __shared__ int64_t best_i[16];
  const T* px = static_cast<const T*>(x);
  const int lane = threadIdx.x % kWave, wave = threadIdx.x / kWave;
  for (int64_t r = blockIdx.x; r < rows; r += gridDim.x) {
    float v = -INFINITY;
    int64_t idx = width;  // sentinel larger than any index
    // kBatch loads in flight per thread (one at a time, a 152k-wide row took 230 us), then
    // the same in-order scan: indices grow, so strict '>' keeps the first maximum
    constexpr int kBatch = 8;
    const int64_t step = blockDim.x;
    for (int64_t i0 = threadIdx.x; i0 < width; i0 += kBatch * step) {
      float e[kBatch];
#pragma unroll
      for (int u = 0; u < kBatch; ++u) {
        const int64_t i = i0 + u * step;
        e[u] = i < width ? ld(px + r * width + i) : -INFINITY;
      }
#pragma unroll
      for (int u = 0; u < kBatch; ++u) {
        const int64_t i = i0 + u * step;
        if (i < width && (e[u] > v || idx == width)) {
          v = e[u];
          idx = i;
        }
      }
    }
#pragma unroll
    for (int off = kWave / 2; off > 0; off >>= 1) {
      const float ov = __shfl_xor(v, off, kWave);
      const int64_t oi = __shfl_xor(idx, off, kWave);
      if (ov > v || (ov == v && oi < idx)) {
        v = ov;
        idx = oi;
      }
    }
    __syncthreads();
    if (lane == 0) {
      best_v[wave] = v;
      best_i[wave] = idx;
    }
    __syncthreads();
    if (threadIdx.x == 0) {
      float bv = best_v[0];
      int64_t bi = best_i[0];
      for (int w = 1; w < static_cast<int>(blockDim.x / kWave); ++w) {
        if (best_v[w] > bv || (best_v[w] == bv && best_i[w] < bi)) {
          bv = best_v[w];
          bi = best_i[w];
        }
      }
      ids[r] = bi < width ? bi : 0;
    }
  }
}

}  // namespace

DK_FLOAT_KERNELS(add, 256, (const void* a, const void* b, void* out, int64_t total, int64_t width),
                 (a, b, out, total, width))
DK_FLOAT_KERNELS(mul, 256, (const void* a, const void* b, void* out, int64_t total, int64_t width),
                 (a, b, out, total, width))
DK_FLOAT_KERNELS(silu, 256, (const void* x, void* out, int64_t total), (x, out, total))
DK_FLOAT_KERNELS(relu, 256, (const void* x, void* out, int64_t total), (x, out, total))
DK_FLOAT_KERNELS(batch_norm2d, 256,
                 (const void* x, const void* w, const void* b, const void* mean, const void* var,
                  void* out, int64_t total, int64_t channels, int64_t spatial, float eps),
                 (x, w, b, mean, var, out, total, channels, spatial, eps))
DK_FLOAT_KERNELS(max_pool2d, 256,
                 (const void* x, void* out, int64_t n, int64_t c, int64_t h, int64_t w, int64_t oh,
                  int64_t ow, int64_t kh, int64_t kw, int64_t sh, int64_t sw, int64_t ph,
                  int64_t pw),
                 (x, out, n, c, h, w, oh, ow, kh, kw, sh, sw, ph, pw))
DK_FLOAT_KERNELS(embedding, 256,
                 (const void* ids, int ids64, const void* table, void* out, int64_t tokens,
                  int64_t hidden, int64_t vocab),
                 (ids, ids64, table, out, tokens, hidden, vocab))
DK_FLOAT_KERNELS(softmax, 256, (const void* x, void* out, int64_t rows, int64_t width),
                 (x, out, rows, width))
DK_FLOAT_KERNELS(transpose2d, 256, (const void* x, void* out, int64_t rows, int64_t cols),
                 (x, out, rows, cols))
DK_FLOAT_KERNELS(rotary, 256,
                 (const void* q, const void* k, const float* cosT, const float* sinT, void* out_q,
                  void* out_k, int64_t batch, int64_t q_heads, int64_t k_heads, int64_t seq,
                  int64_t head_dim, int64_t pairs, int64_t max_pos, int64_t start_pos,
                  const void* positions, int pos64),
                 (q, k, cosT, sinT, out_q, out_k, batch, q_heads, k_heads, seq, head_dim, pairs,
                  max_pos, start_pos, positions, pos64))
DK_FLOAT_KERNELS(argmax, 256, (const void* x, int64_t* ids, int64_t rows, int64_t width),
                 (x, ids, rows, width))

// argmax of fp32 rows whose width is a multiple of 4 on 16-byte aligned rows (vocabulary-wide
// logits): one 1024-thread workgroup per row, 16-byte loads, four in flight per thread (64 KB
// per workgroup, against 8 KB for the generic kernel, whose 152k-wide rows took 67 us for 64
// rows). Each thread scans its elements in index order with the same rule as argmax_impl, and
// the reductions keep the lower index of equal maxima: the first index of the maximum.
extern "C" __global__ void __launch_bounds__(1024)
    argmax_f32_rows_v4(const float* x, int64_t* ids, int64_t rows, int64_t width) {
  typedef float f32x4_t __attribute__((ext_vector_type(4)));
  constexpr int kThreads = 1024, kBatch = 4;
  __shared__ float best_v[kThreads / kWave];
  __shared__ int64_t best_i[kThreads / kWave];
  const int lane = threadIdx.x % kWave, wave = threadIdx.x / kWave;
  const int64_t vecs = width / 4;
  for (int64_t r = blockIdx.x; r < rows; r += gridDim.x) {
    const f32x4_t* row = reinterpret_cast<const f32x4_t*>(x + r * width);
    float v = -INFINITY;
    int64_t idx = width;  // sentinel larger than any index
    for (int64_t j0 = threadIdx.x; j0 < vecs; j0 += kBatch * kThreads) {
      f32x4_t e[kBatch];
#pragma unroll
      for (int u = 0; u < kBatch; ++u) {
        const int64_t j = j0 + u * kThreads;
        e[u] = j < vecs ? *gp(row + j) : f32x4_t{-INFINITY, -INFINITY, -INFINITY, -INFINITY};
      }
#pragma unroll
      for (int u = 0; u < kBatch; ++u) {
        const int64_t j = j0 + u * kThreads;
        if (j >= vecs) break;
#pragma unroll
        for (int c = 0; c < 4; ++c) {
          if (e[u][c] > v || idx == width) {
            v = e[u][c];
            idx = 4 * j + c;
          }
        }
      }
    }
#pragma unroll
    for (int off = kWave / 2; off > 0; off >>= 1) {
      const float ov = __shfl_xor(v, off, kWave);
      const int64_t oi = __shfl_xor(idx, off, kWave);
      if (ov > v || (ov == v && oi < idx)) {
        v = ov;
        idx = oi;
      }
    }
    __syncthreads();
    if (lane == 0) {
      best_v[wave] = v;
      best_i[wave] = idx;
    }
    __syncthreads();
    if (threadIdx.x == 0) {
      float bv = best_v[0];
      int64_t bi = best_i[0];
      for (int w = 1; w < kThreads / kWave; ++w) {
        if (best_v[w] > bv || (best_v[w] == bv && best_i[w] < bi)) {
          bv = best_v[w];
          bi = best_i[w];
        }
      }
      ids[r] = bi < width ? bi : 0;
    }
  }
}

extern "C" __global__ void __launch_bounds__(256)
    permute_0213_u128(const void* x, void* out, int64_t n0, int64_t n1, int64_t n2, int64_t row) {
  typedef uint32_t Chunk16 __attribute__((ext_vector_type(4)));
  permute_0213_impl<Chunk16>(x, out, n0, n1, n2, row);
}
extern "C" __global__ void __launch_bounds__(256)
    permute_0213_u16(const void* x, void* out, int64_t n0, int64_t n1, int64_t n2, int64_t row) {
  permute_0213_impl<uint16_t>(x, out, n0, n1, n2, row);
}
