// Kernel entry points of libdli_hip.so (declared in include/dli_hip.h): argument checks,
// launch geometry, and the launch of the matching embedded gfx950 kernel.
#include <cmath>
#include <string>

#include "../kernels/conv_small.h"
#include "runtime.h"

namespace dli::hip {
namespace {

// The three float variants of one kernel in one code object.
struct FloatKernels {
  DeviceKernel f32, bf16, f16;
  FloatKernels(const char* module, const char* base)
      : f32(module, intern(base, "_f32")), bf16(module, intern(base, "_bf16")),
        f16(module, intern(base, "_f16")) {}

  DeviceKernel* pick(int dtype) {
    switch (dtype) {
      case DLI_F32: return &f32;
      case DLI_BF16: return &bf16;
      case DLI_F16: return &f16;
      default: return nullptr;
    }
  }

 private:
  static const char* intern(const char* base, const char* suffix) {
    return (new std::string(std::string(base) + suffix))->c_str();  // lives for the process
  }
};

int badDtype(const char* op, int dtype) {
  return fail(DLI_HIP_EINVAL, std::string(op) + ": unsupported dtype code " + std::to_string(dtype));
}

int badArg(const char* op, const char* what) {
  return fail(DLI_HIP_EINVAL, std::string(op) + ": " + what);
}

bool validIndexDtype(int dtype) { return dtype == DLI_I64 || dtype == DLI_I32; }

// Grid-stride launches: enough blocks to fill 256 CUs several times over, capped.
unsigned strideBlocks(int64_t work) {
  const int64_t blocks = (work + 255) / 256;
  return static_cast<unsigned>(blocks < 4096 ? (blocks > 0 ? blocks : 1) : 4096);
}

FloatKernels k_add("elementwise", "add");
FloatKernels k_mul("elementwise", "mul");
FloatKernels k_silu("elementwise", "silu");
FloatKernels k_relu("elementwise", "relu");
FloatKernels k_bn("elementwise", "batch_norm2d");
FloatKernels k_maxpool("elementwise", "max_pool2d");
FloatKernels k_embedding("elementwise", "embedding");
FloatKernels k_softmax("elementwise", "softmax");
FloatKernels k_transpose("elementwise", "transpose2d");
DeviceKernel k_permute16("elementwise", "permute_0213_u128");
DeviceKernel k_permute2("elementwise", "permute_0213_u16");
FloatKernels k_rotary("elementwise", "rotary");
FloatKernels k_argmax("elementwise", "argmax");
DeviceKernel k_argmax_rows_v4("elementwise", "argmax_f32_rows_v4");
FloatKernels k_rms_norm("norm", "rms_norm");
DeviceKernel k_rms_norm_rows("norm", "rms_norm_rows_bf16_k");
DeviceKernel k_kv_append_tiles("attention", "kv_append_tiles_bf16_k");
FloatKernels k_gemm("gemm", "gemm_tiled");
DeviceKernel k_skinny1("gemm", "skinny_linear_m1");
DeviceKernel k_skinny2("gemm", "skinny_linear_m2");
DeviceKernel k_skinny4("gemm", "skinny_linear_m4");
FloatKernels k_attention("attention", "attention");
FloatKernels k_paged_attention("attention", "paged_attention");
FloatKernels k_kv_append("attention", "kv_append");
FloatKernels k_conv2d("conv", "conv2d");
DeviceKernel k_flash_attention("flash_attention", "flash_attention_bf16");
DeviceKernel k_flash_attention_q32("flash_attention", "flash_attention_bf16_q32");
DeviceKernel k_mfma_linear64("mfma_gemm", "mfma_linear_f32_t64");
DeviceKernel k_mfma_linear128("mfma_gemm", "mfma_linear_f32_t128");
DeviceKernel k_mfma_matmul64("mfma_gemm", "mfma_matmul_f32_t64");
DeviceKernel k_mfma_matmul128("mfma_gemm", "mfma_matmul_f32_t128");
DeviceKernel k_conv_small9("conv", "conv2d_small_f32_p9");
DeviceKernel k_conv_small27("conv", "conv2d_small_f32_p27");
DeviceKernel k_mfma_conv64("mfma_gemm", "mfma_conv2d_f32_t64");
DeviceKernel k_mfma_conv128("mfma_gemm", "mfma_conv2d_f32_t128");
DeviceKernel k_mfma_bf16_64("mfma_gemm", "mfma_linear_bf16_t64");
DeviceKernel k_mfma_bf16_128("mfma_gemm", "mfma_linear_bf16_t128");
DeviceKernel k_mfma_bf16_splitk("mfma_gemm", "mfma_linear_bf16_splitk_t64");
DeviceKernel k_splitk_reduce_bf16("mfma_gemm", "splitk_reduce_bf16");
DeviceKernel k_mfma_bf16_stream("mfma_gemm", "mfma_linear_bf16_stream_t64");
DeviceKernel k_mfma_linres_stream("mfma_gemm", "mfma_linear_residual_bf16_stream_t64");
DeviceKernel k_mfma_splitk("mfma_gemm", "mfma_linear_f32_splitk_t64");
DeviceKernel k_splitk_reduce("mfma_gemm", "splitk_reduce_f32");
DeviceKernel k_mfma_conv_splitk("mfma_gemm", "mfma_conv2d_f32_splitk_t64");
DeviceKernel k_conv_splitk_reduce("mfma_gemm", "conv_splitk_reduce_f32");

// Split count of an fp32 linear: 64 x 64 tiles are split over K (chunks of at least 256, eight
// 32-wide slices) until there are about 512 workgroups (two per CU); 1 = no split. A workgroup
// walks its K chunk one slice per load round trip, so a few tiles over a long K would otherwise
// take that many round trips.
int64_t linearSplits(int64_t m, int64_t n, int64_t k) {
  const int64_t tiles = ((m + 63) / 64) * ((n + 63) / 64);
  int64_t splits = 1;
  while (splits < 16 && tiles * splits * 2 <= 512 && k / (splits * 2) >= 256) splits *= 2;
  return splits;
}

// MFMA GEMM tiles: 128 x 128 once those alone give every CU a workgroup, else 64 x 64.
bool bigTiles(int64_t rows, int64_t cols) {
  return ((rows + 127) / 128) * ((cols + 127) / 128) >= 256;
}

constexpr int64_t kMaxGridY = 65535;

int binary(FloatKernels& kernels, const char* op, int dtype, const void* a, const void* b,
           void* out, int64_t total, int64_t width, void* stream) {
  DeviceKernel* k = kernels.pick(dtype);
  if (k == nullptr) return badDtype(op, dtype);
  if (total < 0 || width < 0) return badArg(op, "negative size");
  if (total == 0) return 0;
  if (width == 0) return badArg(op, "broadcast operand is empty");
  if (a == nullptr || b == nullptr || out == nullptr) return badArg(op, "NULL pointer");
  return launch(*k, {strideBlocks(total)}, {256}, 0, stream, a, b, out, total, width);
}

int unary(FloatKernels& kernels, const char* op, int dtype, const void* x, void* out,
          int64_t total, void* stream) {
  DeviceKernel* k = kernels.pick(dtype);
  if (k == nullptr) return badDtype(op, dtype);
  if (total < 0) return badArg(op, "negative size");
  if (total == 0) return 0;
  if (x == nullptr || out == nullptr) return badArg(op, "NULL pointer");
  return launch(*k, {strideBlocks(total)}, {256}, 0, stream, x, out, total);
}

bool aligned16(const void* p) { return (reinterpret_cast<uintptr_t>(p) & 15u) == 0; }

}  // namespace

// K splits of the tiled bf16 GEMM for decode-sized m: double while the 64 x 64 tiles times the
// splits stay within 256 workgroups and each part keeps at least 256 columns (at most 16 parts).
// Measured at 64 rows with weights that miss the caches: 3584 x 3584 best at 4 parts (13 us),
// 3584 x 18944 at 4 (33 us), 512 x 3584 at 7-8 (11 us), 18944 x 3584 unsplit (42 us); more
// parts only add fp32 partial traffic.
int64_t bf16Splits(int64_t m, int64_t n, int64_t k) {
  const int64_t tiles = ((m + 63) / 64) * ((n + 63) / 64);
  int64_t splits = 1;
  while (splits < 16 && tiles * splits * 2 <= 256 && k / (splits * 2) >= 256) splits *= 2;
  return splits;
}

// decode-sized bf16 linears that run faster on the tiled MFMA GEMM than on the skinny kernels
// (measured at m = 1, 8, 32, 64 on Qwen2-0.5B and -7B shapes: from m = 64 on every shape, from
// m = 32 on the wide ones, never at m <= 8)
bool tiledDecodeLinear(int64_t m, int64_t n) { return m > 32 || (m > 8 && n >= 8192); }

// The tiled bf16 GEMM over decode-sized m, K split when the workspace allows it: out =
// bf16(x w^T + bias) or, with a residual, bf16(residual + bf16(x w^T + bias)).
int tiledBf16(const void* x, const void* w, const void* bias,
              const void* residual, void* out, int64_t m, int64_t n, int64_t k, void* workspace,
              size_t workspace_bytes, void* stream) {
  int64_t splits = bf16Splits(m, n, k);
  const size_t part = static_cast<size_t>(m * n) * sizeof(float);
  while (splits > 1 && (workspace == nullptr || workspace_bytes < part * splits)) splits /= 2;
  const Dim3 grid{static_cast<unsigned>((n + 63) / 64), static_cast<unsigned>((m + 63) / 64)};
  if (splits == 1) {
    if (residual != nullptr)
      return launch(k_mfma_linres_stream, grid, {256}, 0, stream, x, w, bias, residual, out, m,
                    n, k);
    return launch(k_mfma_bf16_stream, grid, {256}, 0, stream, x, w, bias, out, m, n, k, 0);
  }
  const int64_t per = ((k + splits - 1) / splits + 127) / 128 * 128;  // whole 128-wide slices
  const int64_t parts = (k + per - 1) / per;
  if (int rc = launch(k_mfma_bf16_splitk, {grid.x, grid.y, static_cast<unsigned>(parts)}, {256},
                      0, stream, x, w, static_cast<float*>(workspace), m, n, k, per))
    return rc;
  return launch(k_splitk_reduce_bf16, {strideBlocks(m * n)}, {256}, 0, stream,
                static_cast<const float*>(workspace), bias, residual, out, m, n,
                static_cast<int>(parts));
}

// The split GEMM of tiledBf16 alone: fp32 parts [parts, m, n] of x w^T in the workspace (K in
// whole 128-wide slices over at most bf16Splits(m, n, k) parts, as many as the workspace holds,
// at least one), for a caller's own reduce. *parts_out = the number of parts written.
int tiledBf16Parts(const void* x, const void* w, int64_t m, int64_t n, int64_t k,
                   void* workspace, size_t workspace_bytes, void* stream, int* parts_out) {
  int64_t splits = bf16Splits(m, n, k);
  const size_t part = static_cast<size_t>(m * n) * sizeof(float);
  while (splits > 1 && workspace_bytes < part * splits) splits /= 2;
  if (workspace == nullptr || workspace_bytes < part)
    return fail(DLI_HIP_EINVAL, "tiled split GEMM: workspace too small");
  const int64_t per = ((k + splits - 1) / splits + 127) / 128 * 128;
  const int64_t parts = (k + per - 1) / per;
  *parts_out = static_cast<int>(parts);
  return launch(k_mfma_bf16_splitk,
                {static_cast<unsigned>((n + 63) / 64), static_cast<unsigned>((m + 63) / 64),
                 static_cast<unsigned>(parts)},
                {256}, 0, stream, x, w, static_cast<float*>(workspace), m, n, k, per);
}


int decodeAttentionFast(int dtype, const void* q, const void* key_pool, const void* value_pool,
                        const int32_t* block_table, void* out, int64_t batch, int64_t q_heads,
                        int64_t kv_heads, int64_t seq_q, int64_t head_dim, int64_t block_size,
                        int64_t max_blocks, int64_t past, const void* positions,
                        int positions_dtype, float scale, int requested_splits, void* workspace,
                        size_t workspace_bytes, void* stream);
size_t decodeAttentionWorkspace(int64_t batch, int64_t q_heads, int64_t seq_q, int64_t head_dim,
                                int64_t max_tokens);
}  // namespace dli::hip

using namespace dli::hip;

extern "C" {

int dli_hip_add(int dtype, const void* a, const void* b, void* out, int64_t total, int64_t width,
                void* stream) {
  return binary(k_add, "add", dtype, a, b, out, total, width, stream);
}

int dli_hip_mul(int dtype, const void* a, const void* b, void* out, int64_t total, int64_t width,
                void* stream) {
  return binary(k_mul, "mul", dtype, a, b, out, total, width, stream);
}

int dli_hip_silu(int dtype, const void* x, void* out, int64_t total, void* stream) {
  return unary(k_silu, "silu", dtype, x, out, total, stream);
}

int dli_hip_relu(int dtype, const void* x, void* out, int64_t total, void* stream) {
  return unary(k_relu, "relu", dtype, x, out, total, stream);
}

int dli_hip_rms_norm(int dtype, const void* x, const void* weight, void* out, int64_t rows,
                     int64_t hidden, float eps, void* stream) {
  DeviceKernel* k = k_rms_norm.pick(dtype);
  if (k == nullptr) return badDtype("rms_norm", dtype);
  if (rows < 0 || hidden <= 0) return badArg("rms_norm", "rows must be >= 0 and hidden > 0");
  if (rows == 0) return 0;
  // bf16 rows of up to 4096 elements in 16-byte chunks: one wave per row
  if (dtype == DLI_BF16 && hidden % 8 == 0 && hidden <= 4096 && aligned16(x) &&
      aligned16(weight) && aligned16(out)) {
    const int64_t groups = (rows + 3) / 4;
    const unsigned blocks = static_cast<unsigned>(groups < 65535 ? groups : 65535);
    return launch(k_rms_norm_rows, {blocks}, {256}, 0, stream, x, weight, out, rows,
                  static_cast<int>(hidden), eps);
  }
  const unsigned blocks = static_cast<unsigned>(rows < 65535 ? rows : 65535);
  return launch(*k, {blocks}, {256}, 0, stream, x, weight, out, rows, hidden, eps);
}

int dli_hip_embedding(int dtype, int ids_dtype, const void* ids, const void* table, void* out,
                      int64_t tokens, int64_t hidden, int64_t vocab, void* stream) {
  DeviceKernel* k = k_embedding.pick(dtype);
  if (k == nullptr) return badDtype("embedding", dtype);
  if (!validIndexDtype(ids_dtype)) return badArg("embedding", "ids must be int64 or int32");
  if (tokens < 0 || hidden < 0 || vocab < 0) return badArg("embedding", "negative size");
  if (tokens == 0 || hidden == 0) return 0;
  const int ids64 = ids_dtype == DLI_I64 ? 1 : 0;
  const unsigned blocks = static_cast<unsigned>(tokens < 65535 ? tokens : 65535);
  return launch(*k, {blocks}, {256}, 0, stream, ids, ids64, table, out, tokens, hidden, vocab);
}

int dli_hip_softmax(int dtype, const void* x, void* out, int64_t rows, int64_t width,
                    void* stream) {
  DeviceKernel* k = k_softmax.pick(dtype);
  if (k == nullptr) return badDtype("softmax", dtype);
  if (rows < 0 || width <= 0) return badArg("softmax", "rows must be >= 0 and width > 0");
  if (rows == 0) return 0;
  const unsigned blocks = static_cast<unsigned>(rows < 65535 ? rows : 65535);
  return launch(*k, {blocks}, {256}, 0, stream, x, out, rows, width);
}

int dli_hip_transpose2d(int dtype, const void* x, void* out, int64_t rows, int64_t cols,
                        void* stream) {
  DeviceKernel* k = k_transpose.pick(dtype);
  if (k == nullptr) return badDtype("transpose", dtype);
  if (rows < 0 || cols < 0) return badArg("transpose", "negative size");
  if (rows == 0 || cols == 0) return 0;
  if ((rows + 31) / 32 > 65535) return badArg("transpose", "too many rows");
  return launch(*k, {blocksFor(cols, 32), blocksFor(rows, 32)}, {256}, 0, stream, x, out, rows,
                cols);
}

int dli_hip_permute_0213(int dtype, const void* x, void* out, int64_t n0, int64_t n1, int64_t n2,
                         int64_t n3, void* stream) {
  const char* op = "permute_0213";
  int64_t elem = 0;
  switch (dtype) {
    case DLI_F32: case DLI_I32: elem = 4; break;
    case DLI_BF16: case DLI_F16: elem = 2; break;
    case DLI_I64: elem = 8; break;
    default: return badDtype(op, dtype);
  }
  if (n0 < 0 || n1 < 0 || n2 < 0 || n3 < 0) return badArg(op, "negative size");
  if (n0 == 0 || n1 == 0 || n2 == 0 || n3 == 0) return 0;
  if (x == nullptr || out == nullptr) return badArg(op, "NULL pointer");
  const int64_t row_bytes = n3 * elem;
  const bool wide = row_bytes % 16 == 0 && (reinterpret_cast<uintptr_t>(x) & 15u) == 0 &&
                    (reinterpret_cast<uintptr_t>(out) & 15u) == 0;
  const int64_t row = wide ? row_bytes / 16 : row_bytes / 2;
  return launch(wide ? k_permute16 : k_permute2, {strideBlocks(n0 * n1 * n2 * row)}, {256}, 0,
                stream, x, out, n0, n1, n2, row);
}

int dli_hip_batch_norm2d(int dtype, const void* x, const void* weight, const void* bias,
                         const void* running_mean, const void* running_var, void* out,
                         int64_t total, int64_t channels, int64_t spatial, float eps,
                         void* stream) {
  DeviceKernel* k = k_bn.pick(dtype);
  if (k == nullptr) return badDtype("batch_norm2d", dtype);
  if (total < 0 || channels <= 0 || spatial <= 0)
    return badArg("batch_norm2d", "channels and spatial must be positive");
  if (total == 0) return 0;
  return launch(*k, {strideBlocks(total)}, {256}, 0, stream, x, weight, bias, running_mean,
                running_var, out, total, channels, spatial, eps);
}

int dli_hip_max_pool2d(int dtype, const void* x, void* out, int64_t n, int64_t c, int64_t h,
                       int64_t w, int64_t out_h, int64_t out_w, int64_t kernel_h,
                       int64_t kernel_w, int64_t stride_h, int64_t stride_w, int64_t pad_h,
                       int64_t pad_w, void* stream) {
  DeviceKernel* k = k_maxpool.pick(dtype);
  if (k == nullptr) return badDtype("max_pool2d", dtype);
  if (kernel_h <= 0 || kernel_w <= 0 || stride_h <= 0 || stride_w <= 0 || pad_h < 0 || pad_w < 0)
    return badArg("max_pool2d", "kernel and stride must be positive, padding non-negative");
  const int64_t total = n * c * out_h * out_w;
  if (n < 0 || c < 0 || out_h < 0 || out_w < 0) return badArg("max_pool2d", "negative size");
  if (total == 0) return 0;
  return launch(*k, {strideBlocks(total)}, {256}, 0, stream, x, out, n, c, h, w, out_h, out_w,
                kernel_h, kernel_w, stride_h, stride_w, pad_h, pad_w);
}

int dli_hip_conv2d(int dtype, const void* x, const void* weight, const void* bias, void* out,
                   int64_t n, int64_t in_c, int64_t h, int64_t w, int64_t out_c, int64_t kernel_h,
                   int64_t kernel_w, int64_t out_h, int64_t out_w, int64_t stride_h,
                   int64_t stride_w, int64_t pad_h, int64_t pad_w, void* stream) {
  return dli_hip_conv2d_act(dtype, x, weight, bias, out, n, in_c, h, w, out_c, kernel_h, kernel_w,
                            out_h, out_w, stride_h, stride_w, pad_h, pad_w, DLI_ACT_NONE, nullptr,
                            0, stream);
}

size_t dli_hip_conv2d_workspace(int dtype, int64_t n, int64_t in_c, int64_t out_c,
                                int64_t kernel_h, int64_t kernel_w, int64_t out_h, int64_t out_w) {
  if (dtype != DLI_F32 || n <= 0 || in_c <= 0 || out_c <= 0 || kernel_h <= 0 || kernel_w <= 0 ||
      out_h <= 0 || out_w <= 0)
    return 0;
  const int64_t pixels = n * out_h * out_w;
  if (bigTiles(out_c, pixels)) return 0;
  const int64_t splits = linearSplits(out_c, pixels, in_c * kernel_h * kernel_w);
  return splits > 1 ? static_cast<size_t>(splits * out_c * pixels) * sizeof(float) : 0;
}

int dli_hip_conv2d_act(int dtype, const void* x, const void* weight, const void* bias, void* out,
                       int64_t n, int64_t in_c, int64_t h, int64_t w, int64_t out_c,
                       int64_t kernel_h, int64_t kernel_w, int64_t out_h, int64_t out_w,
                       int64_t stride_h, int64_t stride_w, int64_t pad_h, int64_t pad_w,
                       int activation, void* workspace, size_t workspace_bytes, void* stream) {
  if (activation != DLI_ACT_NONE && activation != DLI_ACT_RELU)
    return badArg("conv2d", "unknown activation");
  if (stride_h <= 0 || stride_w <= 0 || pad_h < 0 || pad_w < 0)
    return badArg("conv2d", "stride must be positive, padding non-negative");
  if (n < 0 || in_c < 0 || out_c < 0 || out_h < 0 || out_w < 0 || h < 0 || w < 0 ||
      kernel_h < 0 || kernel_w < 0)
    return badArg("conv2d", "negative size");
  const int64_t total = n * out_c * out_h * out_w;
  if (total == 0) return 0;
  if (x == nullptr || weight == nullptr || out == nullptr) return badArg("conv2d", "NULL pointer");
  const int relu = activation == DLI_ACT_RELU ? 1 : 0;
  // fp32: implicit GEMM on MFMA, 32-bit index math (every element index below 2^31)
  const int64_t pixels = n * out_h * out_w, patch = in_c * kernel_h * kernel_w;
  const int64_t limit = int64_t{1} << 31;
  if (dtype == DLI_F32 && kernel_h < 65536 && kernel_w < 65536 && n * in_c * h * w < limit &&
      total < limit && out_c * patch < limit &&
      pixels < limit && (out_h - 1) * stride_h + kernel_h < limit &&
      (out_w - 1) * stride_w + kernel_w < limit) {
    auto i32 = [](int64_t v) { return static_cast<int>(v); };
    // a patch too short for MFMA tiles (an RGB input layer): direct, output-write bound
    if ((patch == 9 || patch == 27) && (out_c + dk::kSmallOc - 1) / dk::kSmallOc <= kMaxGridY) {
      dk::SmallConvTable tab{};
      tab.patch = i32(patch);
      for (int k = 0; k < tab.patch; ++k) {
        const int c = k / i32(kernel_h * kernel_w), ky = (k / i32(kernel_w)) % i32(kernel_h),
                  kx = k % i32(kernel_w);
        tab.offset[k] = (c * i32(h) + ky) * i32(w) + kx;
        tab.ky[k] = ky;
        tab.kx[k] = kx;
      }
      return launch(patch == 9 ? k_conv_small9 : k_conv_small27,
                    {static_cast<unsigned>((pixels + 255) / 256),
                     static_cast<unsigned>((out_c + dk::kSmallOc - 1) / dk::kSmallOc)},
                    {256}, 0, stream, x, weight, bias, out, i32(n), i32(in_c), i32(h), i32(w),
                    i32(out_c), i32(out_h), i32(out_w), i32(stride_h), i32(stride_w), i32(pad_h),
                    i32(pad_w), relu, tab);
    }
    const bool big = bigTiles(out_c, pixels);
    const int64_t tile = big ? 128 : 64;
    const int64_t splits = big ? 1 : linearSplits(out_c, pixels, patch);
    const size_t need = static_cast<size_t>(splits * out_c * pixels) * sizeof(float);
    if (splits > 1 && workspace != nullptr && workspace_bytes >= need &&
        (out_c + 63) / 64 <= kMaxGridY) {
      const int64_t per = (patch + splits - 1) / splits;
      int rc = launch(k_mfma_conv_splitk,
                      {static_cast<unsigned>((pixels + 63) / 64),
                       static_cast<unsigned>((out_c + 63) / 64), static_cast<unsigned>(splits)},
                      {256}, 0, stream, x, weight, workspace, i32(n), i32(in_c), i32(h), i32(w),
                      i32(out_c), i32(kernel_h), i32(kernel_w), i32(out_h), i32(out_w),
                      i32(stride_h), i32(stride_w), i32(pad_h), i32(pad_w), i32(per));
      if (rc != 0) return rc;
      return launch(k_conv_splitk_reduce, {strideBlocks(out_c * pixels)}, {256}, 0, stream,
                    workspace, bias, out, out_c, pixels, out_h * out_w,
                    static_cast<int>(splits), relu);
    }
    if ((out_c + tile - 1) / tile <= kMaxGridY) {
      return launch(big ? k_mfma_conv128 : k_mfma_conv64,
                    {static_cast<unsigned>((pixels + tile - 1) / tile),
                     static_cast<unsigned>((out_c + tile - 1) / tile)},
                    {256}, 0, stream, x, weight, bias, out, i32(n), i32(in_c), i32(h), i32(w),
                    i32(out_c), i32(kernel_h), i32(kernel_w), i32(out_h), i32(out_w),
                    i32(stride_h), i32(stride_w), i32(pad_h), i32(pad_w), relu);
    }
  }
  DeviceKernel* k = k_conv2d.pick(dtype);
  if (k == nullptr) return badDtype("conv2d", dtype);
  int rc = launch(*k, {strideBlocks(total)}, {256}, 0, stream, x, weight, bias, out, n, in_c, h, w,
                  out_c, kernel_h, kernel_w, out_h, out_w, stride_h, stride_w, pad_h, pad_w);
  if (rc == 0 && relu) rc = unary(k_relu, "relu", dtype, out, out, total, stream);
  return rc;
}

int dli_hip_linear(int dtype, int out_dtype, const void* x, const void* w, const void* bias,
                   void* out, int64_t m, int64_t n, int64_t k, void* stream) {
  return dli_hip_linear_act(dtype, out_dtype, x, w, bias, out, m, n, k, DLI_ACT_NONE, nullptr, 0,
                            stream);
}

size_t dli_hip_linear_workspace(int dtype, int64_t m, int64_t n, int64_t k) {
  if (m <= 0 || n <= 0 || k <= 0) return 0;
  if (dtype == DLI_BF16) {  // decode-sized m on the tiled GEMM: K split over fp32 parts
    if (m > 64 || !tiledDecodeLinear(m, n) || k % 8 != 0) return 0;  // (fp32-out calls ignore it)
    const int64_t splits = bf16Splits(m, n, k);
    return splits > 1 ? static_cast<size_t>(splits * m * n) * sizeof(float) : 0;
  }
  if (dtype != DLI_F32) return 0;
  const int64_t splits = linearSplits(m, n, k);
  return splits > 1 ? static_cast<size_t>(splits * m * n) * sizeof(float) : 0;
}

int dli_hip_linear_act(int dtype, int out_dtype, const void* x, const void* w, const void* bias,
                       void* out, int64_t m, int64_t n, int64_t k, int activation,
                       void* workspace, size_t workspace_bytes, void* stream) {
  if (activation != DLI_ACT_NONE && activation != DLI_ACT_RELU)
    return badArg("linear", "unknown activation");
  if (out_dtype != dtype && out_dtype != DLI_F32)
    return badArg("linear", "out_dtype must equal dtype or be float32");
  if (m < 0 || n < 0 || k < 0) return badArg("linear", "negative size");
  if (m == 0 || n == 0) return 0;
  if (x == nullptr || w == nullptr || out == nullptr) return badArg("linear", "NULL pointer");
  const int out_f32 = out_dtype == DLI_F32 ? 1 : 0;
  const int relu = activation == DLI_ACT_RELU ? 1 : 0;
  const bool big = bigTiles(m, n);
  const int64_t tile = big ? 128 : 64;
  const Dim3 grid{static_cast<unsigned>((n + tile - 1) / tile),
                  static_cast<unsigned>((m + tile - 1) / tile)};
  const bool grid_ok = (m + tile - 1) / tile <= kMaxGridY;
  if (dtype == DLI_F32 && grid_ok) {
    const int64_t splits = linearSplits(m, n, k);
    const size_t need = static_cast<size_t>(splits * m * n) * sizeof(float);
    if (splits > 1 && workspace != nullptr && workspace_bytes >= need) {
      const int64_t per = (k + splits - 1) / splits;
      int rc = launch(k_mfma_splitk,
                      {static_cast<unsigned>((n + 63) / 64), static_cast<unsigned>((m + 63) / 64),
                       static_cast<unsigned>(splits)},
                      {256}, 0, stream, x, w, workspace, m, n, k, per);
      if (rc != 0) return rc;
      return launch(k_splitk_reduce, {strideBlocks(m * n)}, {256}, 0, stream, workspace, bias,
                    out, m, n, static_cast<int>(splits), relu);
    }
    return launch(big ? k_mfma_linear128 : k_mfma_linear64, grid, {256}, 0, stream, x, w, bias,
                  out, m, n, k, relu);
  }
  int rc;
  if (dtype == DLI_BF16 && m <= 64 && tiledDecodeLinear(m, n) && k % 8 == 0 && aligned16(x) &&
      aligned16(w) && !relu) {
    if (out_f32)  // fp32 logits: one pass, no split (the split reduce writes bf16)
      return launch(k_mfma_bf16_stream,
                    {static_cast<unsigned>((n + 63) / 64), static_cast<unsigned>((m + 63) / 64)},
                    {256}, 0, stream, x, w, bias, out, m, n, k, out_f32);
    return tiledBf16(x, w, bias, nullptr, out, m, n, k, workspace, workspace_bytes,
                     stream);
  } else if (dtype == DLI_BF16 && m <= 64 && k % 64 == 0 && aligned16(x) && aligned16(w)) {
    // bf16 weight streaming for decode-sized m: MFMA skinny kernel.
    DeviceKernel* sk = m <= 16 ? &k_skinny1 : (m <= 32 ? &k_skinny2 : &k_skinny4);
    rc = launch(*sk, {blocksFor(n, 32)}, {256}, 0, stream, x, w, bias, out, m, n, k, out_f32);
  } else if (dtype == DLI_BF16 && k % 8 == 0 && aligned16(x) && aligned16(w) &&
             (m + 63) / 64 <= kMaxGridY) {
    // the bf16 GEMM's own tile rule (its 128 x 128 tiles pay off from about 168 of them)
    const bool b128 = ((m + 127) / 128) * ((n + 127) / 128) >= 168;
    const int64_t bt = b128 ? 128 : 64;
    return launch(b128 ? k_mfma_bf16_128 : k_mfma_bf16_64,
                  {static_cast<unsigned>((n + bt - 1) / bt), static_cast<unsigned>((m + bt - 1) / bt)},
                  {256}, 0, stream, x, w, bias, out, m, n, k, out_f32, relu);
  } else {
    DeviceKernel* kt = k_gemm.pick(dtype);
    if (kt == nullptr) return badDtype("linear", dtype);
    if ((m + 63) / 64 > kMaxGridY) return badArg("linear", "m too large");
    rc = launch(*kt, {blocksFor(n, 64), blocksFor(m, 64)}, {256}, 0, stream, x, w, bias, out, m,
                n, k, 1, out_f32);
  }
  if (rc == 0 && relu) rc = unary(k_relu, "relu", out_dtype, out, out, m * n, stream);
  return rc;
}

int dli_hip_matmul(int dtype, const void* a, const void* b, void* out, int64_t m, int64_t n,
                   int64_t k, void* stream) {
  if (m < 0 || n < 0 || k < 0) return badArg("matmul", "negative size");
  if (m == 0 || n == 0) return 0;
  if (a == nullptr || b == nullptr || out == nullptr) return badArg("matmul", "NULL pointer");
  const bool big = bigTiles(m, n);
  const int64_t tile = big ? 128 : 64;
  if (dtype == DLI_F32 && (m + tile - 1) / tile <= kMaxGridY)
    return launch(big ? k_mfma_matmul128 : k_mfma_matmul64,
                  {static_cast<unsigned>((n + tile - 1) / tile),
                   static_cast<unsigned>((m + tile - 1) / tile)},
                  {256}, 0, stream, a, b, out, m, n, k);
  DeviceKernel* kt = k_gemm.pick(dtype);
  if (kt == nullptr) return badDtype("matmul", dtype);
  if ((m + 63) / 64 > kMaxGridY) return badArg("matmul", "m too large");
  const void* no_bias = nullptr;
  return launch(*kt, {blocksFor(n, 64), blocksFor(m, 64)}, {256}, 0, stream, a, b, no_bias, out, m,
                n, k, 0, 0);
}

int dli_hip_rotary(int dtype, const void* q, const void* k, const float* cos_table,
                   const float* sin_table, void* out_q, void* out_k, int64_t batch,
                   int64_t q_heads, int64_t k_heads, int64_t seq, int64_t head_dim, int64_t pairs,
                   int64_t max_pos, int64_t start_pos, const void* positions,
                   int positions_dtype, void* stream) {
  DeviceKernel* kr = k_rotary.pick(dtype);
  if (kr == nullptr) return badDtype("rotary_embedding", dtype);
  if (head_dim <= 0 || head_dim % 2 != 0) return badArg("rotary_embedding", "head_dim must be even");
  if (pairs < 0 || 2 * pairs > head_dim) return badArg("rotary_embedding", "pairs > head_dim / 2");
  if (positions != nullptr && !validIndexDtype(positions_dtype))
    return badArg("rotary_embedding", "positions must be int64 or int32");
  if (batch < 0 || q_heads < 0 || k_heads < 0 || seq < 0) return badArg("rotary_embedding", "negative size");
  const int64_t work = batch * (q_heads > k_heads ? q_heads : k_heads) * seq * (head_dim / 2);
  if (work == 0) return 0;
  const int pos64 = positions_dtype == DLI_I64 ? 1 : 0;
  return launch(*kr, {strideBlocks(work)}, {256}, 0, stream, q, k, cos_table, sin_table, out_q,
                out_k, batch, q_heads, k_heads, seq, head_dim, pairs, max_pos, start_pos, positions,
                pos64);
}

// attention with out as [B, Hq, Sq, D] (out_bshd 0) or [B, Sq, Hq, D] (1, flash path only)
static int attentionImpl(int dtype, const void* q, const void* k, const void* v, void* out,
                  int64_t batch, int64_t q_heads, int64_t kv_heads, int64_t seq_q, int64_t seq_k,
                  int64_t head_dim, int causal, float scale, int out_bshd, void* stream) {
  DeviceKernel* ka = k_attention.pick(dtype);
  if (ka == nullptr) return badDtype("attention", dtype);
  if (head_dim <= 0 || head_dim > 256) return badArg("attention", "head_dim must be in [1, 256]");
  if (kv_heads <= 0 || q_heads % kv_heads != 0)
    return badArg("attention", "q_heads must be a multiple of kv_heads");
  if (batch < 0 || seq_q < 0 || seq_k < 0) return badArg("attention", "negative size");
  const int64_t rows = batch * q_heads * seq_q;
  if (rows == 0) return 0;
  if (q == nullptr || k == nullptr || v == nullptr || out == nullptr)
    return badArg("attention", "NULL pointer");
  // bf16 with head_dim 64 (prefill): flash-style MFMA kernel, 128 queries per workgroup (64 for
  // query sequences of at most 64)
  if (dtype == DLI_BF16 && head_dim == 64 && seq_k > 0 && batch * q_heads <= 65535 &&
      seq_q < (int64_t{1} << 30) && seq_k < (int64_t{1} << 30) &&
      aligned16(q) && aligned16(k) && aligned16(v) && aligned16(out)) {
    const float log2e = 1.4426950408889634f;
    const int64_t tile_q = seq_q > 64 ? 128 : 64;
    return launch(tile_q == 128 ? k_flash_attention_q32 : k_flash_attention,
                  {static_cast<unsigned>((seq_q + tile_q - 1) / tile_q),
                   static_cast<unsigned>(batch * q_heads)},
                  {256}, 0, stream, q, k, v, out, q_heads, kv_heads, seq_q, seq_k, causal,
                  scale * log2e, out_bshd);
  }
  if (out_bshd)
    return badArg("attention", "a [B, S, H, D] output needs bf16, head_dim 64, seq_k > 0 and "
                               "16-byte aligned tensors (the flash kernel)");
  if (rows > 0x7fffffff) return badArg("attention", "too many query rows");
  return launch(*ka, {static_cast<unsigned>(rows)}, {64}, 0, stream, q, k, v, out, batch, q_heads,
                kv_heads, seq_q, seq_k, head_dim, causal, scale);
}

int dli_hip_attention(int dtype, const void* q, const void* k, const void* v, void* out,
                      int64_t batch, int64_t q_heads, int64_t kv_heads, int64_t seq_q,
                      int64_t seq_k, int64_t head_dim, int causal, float scale, void* stream) {
  return attentionImpl(dtype, q, k, v, out, batch, q_heads, kv_heads, seq_q, seq_k, head_dim,
                       causal, scale, 0, stream);
}

int dli_hip_attention_bshd(int dtype, const void* q, const void* k, const void* v, void* out,
                           int64_t batch, int64_t q_heads, int64_t kv_heads, int64_t seq_q,
                           int64_t seq_k, int64_t head_dim, int causal, float scale,
                           void* stream) {
  return attentionImpl(dtype, q, k, v, out, batch, q_heads, kv_heads, seq_q, seq_k, head_dim,
                       causal, scale, 1, stream);
}

int dli_hip_kv_append(int dtype, const void* key, const void* value, void* key_pool,
                      void* value_pool, const int32_t* block_table, int64_t batch, int64_t heads,
                      int64_t seq, int64_t head_dim, int64_t block_size, int64_t max_blocks,
                      int64_t start, const void* positions, int positions_dtype, void* stream) {
  DeviceKernel* ka = k_kv_append.pick(dtype);
  if (ka == nullptr) return badDtype("kv_append", dtype);
  if (block_size <= 0 || max_blocks <= 0) return badArg("kv_append", "empty cache geometry");
  if (positions != nullptr && !validIndexDtype(positions_dtype))
    return badArg("kv_append", "positions must be int64 or int32");
  if (batch < 0 || heads < 0 || seq < 0 || head_dim < 0) return badArg("kv_append", "negative size");
  const int64_t total = batch * heads * seq * head_dim;
  if (total == 0) return 0;
  const int pos64 = positions_dtype == DLI_I64 ? 1 : 0;
  // bf16 prompts (at least 16 new tokens) with 16-byte rows: 64 tokens of one head per
  // workgroup, values transposed in LDS (a decode step's one token stays on the element kernel:
  // 14 us against a few for the tiles at batch 64 x 4 heads)
  if (dtype == DLI_BF16 && seq >= 16 && head_dim % 8 == 0 && head_dim <= 256 &&
      batch * heads <= 65535 &&
      aligned16(key) && aligned16(value) && aligned16(key_pool)) {
    const int64_t chunks = (seq + 63) / 64;
    if (chunks <= 0x7fffffff)
      return launch(k_kv_append_tiles, {static_cast<unsigned>(chunks),
                                        static_cast<unsigned>(batch * heads)},
                    {256}, 0, stream, key, value, key_pool, value_pool, block_table, heads, seq,
                    static_cast<int>(head_dim), block_size, max_blocks, start, positions, pos64);
  }
  return launch(*ka, {strideBlocks(total)}, {256}, 0, stream, key, value, key_pool, value_pool,
                block_table, batch, heads, seq, head_dim, block_size, max_blocks, start, positions,
                pos64);
}

size_t dli_hip_paged_attention_workspace(int64_t batch, int64_t q_heads, int64_t seq_q,
                                         int64_t head_dim, int64_t max_tokens) {
  return decodeAttentionWorkspace(batch, q_heads, seq_q, head_dim, max_tokens);
}

int dli_hip_paged_attention(int dtype, const void* q, const void* key_pool,
                            const void* value_pool, const int32_t* block_table, void* out,
                            int64_t batch, int64_t q_heads, int64_t kv_heads, int64_t seq_q,
                            int64_t head_dim, int64_t block_size, int64_t max_blocks, int64_t past,
                            const void* positions, int positions_dtype, int causal, float scale,
                            int splits, void* workspace, size_t workspace_bytes, void* stream) {
  DeviceKernel* ka = k_paged_attention.pick(dtype);
  if (ka == nullptr) return badDtype("paged_attention", dtype);
  if (head_dim <= 0 || head_dim > 256) return badArg("paged_attention", "head_dim must be in [1, 256]");
  if (kv_heads <= 0 || q_heads % kv_heads != 0)
    return badArg("paged_attention", "q_heads must be a multiple of kv_heads");
  if (block_size <= 0 || max_blocks <= 0) return badArg("paged_attention", "empty cache geometry");
  if (positions != nullptr && !validIndexDtype(positions_dtype))
    return badArg("paged_attention", "positions must be int64 or int32");
  if (batch < 0 || seq_q < 0) return badArg("paged_attention", "negative size");
  if (splits < 0 || splits > kMaxDecodeSplits)
    return badArg("paged_attention", "splits must be in [0, 32]");
  const int64_t rows = batch * q_heads * seq_q;
  if (rows == 0) return 0;
  if (rows > 0x7fffffff) return badArg("paged_attention", "too many query rows");
  if (causal || seq_q == 1) {
    const int rc = decodeAttentionFast(dtype, q, key_pool, value_pool, block_table, out, batch,
                                       q_heads, kv_heads, seq_q, head_dim, block_size, max_blocks,
                                       past, positions, positions_dtype, scale, splits, workspace,
                                       workspace_bytes, stream);
    if (rc != 1) return rc;
  }
  const int pos64 = positions_dtype == DLI_I64 ? 1 : 0;
  return launch(*ka, {static_cast<unsigned>(rows)}, {64}, 0, stream, q, key_pool, value_pool,
                block_table, out, batch, q_heads, kv_heads, seq_q, head_dim, block_size, max_blocks,
                past, positions, pos64, causal, scale);
}

int dli_hip_argmax(int dtype, const void* x, int64_t* ids, int64_t rows, int64_t width,
                   void* stream) {
  DeviceKernel* ka = k_argmax.pick(dtype);
  if (ka == nullptr) return badDtype("argmax", dtype);
  if (rows < 0 || width <= 0) return badArg("argmax", "rows must be >= 0 and width > 0");
  if (rows == 0) return 0;
  const unsigned blocks = static_cast<unsigned>(rows < 65535 ? rows : 65535);
  // wide fp32 rows (logits over a vocabulary): the 16-byte-load kernel
  if (dtype == DLI_F32 && width % 4 == 0 && width >= 4096 &&
      (reinterpret_cast<uintptr_t>(x) & 15u) == 0)
    return launch(k_argmax_rows_v4, {blocks}, {1024}, 0, stream, x, ids, rows, width);
  return launch(*ka, {blocks}, {256}, 0, stream, x, ids, rows, width);
}

}  // extern "C"
