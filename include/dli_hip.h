/*
 * dli_hip.h — C ABI of libdli_hip.so, the MI355X (gfx950) device layer of dl-inference.
 *
 * Plain C: pointers, sizes and int status codes only (no torch or C++ types), so it can be
 * bound from ctypes, cgo or any other FFI. Two groups of entry points:
 *
 *  1. Launch / allocator layer. Replaces the dlopen'd CUDA driver and runtime wrappers of
 *     the reference: include/dli/cuda_driver.h:8-32 (CudaAotKernel: cuModuleLoadData,
 *     cuModuleGetFunction, cuLaunchKernel) and include/dli/cuda_runtime.h:8-18
 *     (cudaMallocBytes / cudaFreePointer / cudaMemcpyBytes). The HIP runtime is dlopen'd on
 *     first use; without a GPU the calls fail with an error text instead of aborting.
 *
 *  2. Kernel entry points, one per operator of the reference plugin, plus fused decode
 *     kernels. Each replaces the argument packing + cuLaunchKernel of one
 *     python/dli_ops/aot/<op>/template.cc and follows the semantics of the matching
 *     python/dli_ops/aot/<op>/kernel.py (cited per function). Kernels are hand-written HIP
 *     for gfx950, compiled ahead of time to code objects embedded in the library.
 *
 * Conventions
 *  - Return value: 0 on success; DLI_HIP_EINVAL (-1) for a rejected argument, DLI_HIP_ENODEV
 *    (-2) when no HIP runtime/device is usable, otherwise the hipError_t code. The message of
 *    the last failure on the calling thread is returned by dli_hip_last_error().
 *  - stream: a hipStream_t passed as void*; NULL is the null stream. Every kernel entry point
 *    is asynchronous on that stream, allocates nothing and never synchronizes, so a sequence
 *    of them can be captured into a HIP graph.
 *  - dtype codes follow dli::DType: DLI_F32=0, DLI_I64=1, DLI_BF16=2, DLI_F16=3, DLI_I32=4.
 *    Floating kernels compute in fp32 and round the result to the output dtype once.
 *  - Sizes are element counts unless named *_bytes. Zero-sized work is a successful no-op.
 */
#ifndef DLI_HIP_H_
#define DLI_HIP_H_

#include <stddef.h>
#include <stdint.h>

#ifdef __cplusplus
extern "C" {
#endif

enum {
  DLI_F32 = 0,
  DLI_I64 = 1,
  DLI_BF16 = 2,
  DLI_F16 = 3,
  DLI_I32 = 4,
};

enum {
  DLI_HIP_OK = 0,
  DLI_HIP_EINVAL = -1,
  DLI_HIP_ENODEV = -2,
};

/* Activations fused into a GEMM epilogue (dli_hip_linear_act, dli_hip_conv2d_act). */
enum {
  DLI_ACT_NONE = 0,
  DLI_ACT_RELU = 1,
};

/* memcpy kinds, numbered as cudaMemcpyKind in include/dli/cuda_runtime.h:8-12. */
enum {
  DLI_MEMCPY_HOST_TO_DEVICE = 1,
  DLI_MEMCPY_DEVICE_TO_HOST = 2,
  DLI_MEMCPY_DEVICE_TO_DEVICE = 3,
};

/* ---------------------------------------------------------------------------------------
 * 1. Launch / allocator layer
 * ------------------------------------------------------------------------------------- */

/* 1 when the HIP runtime loaded and reports at least one device (cuda_driver.h:8). */
int dli_hip_available(void);
/* Why the runtime is unavailable; "" when it is available (cuda_driver.h:9). */
const char* dli_hip_load_error(void);
/* Message of the last failed dli_hip_* call on this thread. */
const char* dli_hip_last_error(void);
/* Architecture the embedded code objects were built for, e.g. "gfx950". */
const char* dli_hip_target_arch(void);

int dli_hip_device_count(int* count);
int dli_hip_get_device(int* device);
/* Compute units of the current device (hipDeviceAttributeMultiprocessorCount; the reference
 * has no counterpart: its launch grids do not depend on the device). */
int dli_hip_compute_units(int* count);
int dli_hip_set_device(int device);

/* Module load + launch (CudaAotKernel::load / launch, cuda_driver.cc:107-129). A launch with
 * any grid dimension 0 returns 0 without touching the runtime (cuda_driver.cc:123). */
int dli_hip_module_load(const void* image, size_t image_bytes, void** module);
/* Image of the library's embedded gfx950 code object `name` ("attention", "conv", "decode",
 * "elementwise", "flash_attention", "gemm", "mfma_gemm", "norm", "stack"), for
 * dli_hip_module_load. The reference's counterpart is the cubin file its plugin reads next to
 * itself (CudaAotKernel::load, cuda_driver.cc:107-117); here the images live inside the library.
 * The image stays valid while the library is loaded. */
int dli_hip_code_object(const char* name, const void** image, size_t* image_bytes);
int dli_hip_module_get_function(void* module, const char* name, void** function);
int dli_hip_module_unload(void* module);
int dli_hip_launch(void* function, unsigned grid_x, unsigned grid_y, unsigned grid_z,
                   unsigned block_x, unsigned block_y, unsigned block_z, unsigned lds_bytes,
                   void* stream, void** args);

/* Allocator / copies (cuda_runtime.cc:74-91). dli_hip_free(NULL) is a no-op. */
int dli_hip_malloc(size_t bytes, void** ptr);
int dli_hip_free(void* ptr);
int dli_hip_memcpy(void* dst, const void* src, size_t bytes, int kind);
int dli_hip_memcpy_async(void* dst, const void* src, size_t bytes, int kind, void* stream);
int dli_hip_stream_synchronize(void* stream);
int dli_hip_device_synchronize(void);

/* Events for timing kernels on a given stream. */
int dli_hip_event_create(void** event);
int dli_hip_event_record(void* event, void* stream);
int dli_hip_event_synchronize(void* event);
int dli_hip_event_elapsed_ms(void* start, void* stop, float* ms);
int dli_hip_event_destroy(void* event);
/* *capturing = 1 while `stream` is being captured into a graph (or its capture was
 * invalidated), else 0. */
int dli_hip_stream_is_capturing(void* stream, int* capturing);

/* ---------------------------------------------------------------------------------------
 * 2. Kernel entry points
 * ------------------------------------------------------------------------------------- */

/* out[i] = a[i] + b[i % width] (add/kernel.py:6-11; add/template.cc:10-14). */
int dli_hip_add(int dtype, const void* a, const void* b, void* out, int64_t total,
                int64_t width, void* stream);
/* out[i] = a[i] * b[i % width] (mul/kernel.py:6-11; mul/template.cc:10-14). */
int dli_hip_mul(int dtype, const void* a, const void* b, void* out, int64_t total,
                int64_t width, void* stream);
/* out = x / (1 + exp(-x)) (silu/kernel.py:6-10). */
int dli_hip_silu(int dtype, const void* x, void* out, int64_t total, void* stream);
/* out = max(x, 0) (relu/kernel.py:6-10). */
int dli_hip_relu(int dtype, const void* x, void* out, int64_t total, void* stream);

/* y = x * rsqrt(mean(x^2) + eps) * w per row of `hidden` (rms_norm/kernel.py:6-14;
 * rms_norm/template.cc:20-26). x, w, out share dtype. */
int dli_hip_rms_norm(int dtype, const void* x, const void* weight, void* out, int64_t rows,
                     int64_t hidden, float eps, void* stream);

/* out[t, :] = table[ids[t], :] (embedding/kernel.py:6-23). ids_dtype is DLI_I64 or DLI_I32.
 * An id outside [0, vocab) yields a zero row. */
int dli_hip_embedding(int dtype, int ids_dtype, const void* ids, const void* table, void* out,
                      int64_t tokens, int64_t hidden, int64_t vocab, void* stream);

/* Row softmax over the last dim (softmax/kernel.py:6-14), any width. */
int dli_hip_softmax(int dtype, const void* x, void* out, int64_t rows, int64_t width,
                    void* stream);

/* out[c, r] = x[r, c] (transpose/kernel.py:6-20). */
int dli_hip_transpose2d(int dtype, const void* x, void* out, int64_t rows, int64_t cols,
                        void* stream);

/* out[a, c, b, :] = x[a, b, c, :] for x [n0, n1, n2, n3] (permutation [0, 2, 1, 3]): the
 * [B, S, H, D] <-> [B, H, S, D] layout change of a prefill graph. Extends the reference's
 * transpose (transpose/kernel.py:6-20, 2-D only); any dtype code (a copy). */
int dli_hip_permute_0213(int dtype, const void* x, void* out, int64_t n0, int64_t n1, int64_t n2,
                         int64_t n3, void* stream);

/* Eval batch norm on NCHW (batch_norm2d/kernel.py:6-28). */
int dli_hip_batch_norm2d(int dtype, const void* x, const void* weight, const void* bias,
                         const void* running_mean, const void* running_var, void* out,
                         int64_t total, int64_t channels, int64_t spatial, float eps,
                         void* stream);

/* Max pooling with -inf padding on NCHW (max_pool2d/kernel.py:6-41). */
int dli_hip_max_pool2d(int dtype, const void* x, void* out, int64_t n, int64_t c, int64_t h,
                       int64_t w, int64_t out_h, int64_t out_w, int64_t kernel_h,
                       int64_t kernel_w, int64_t stride_h, int64_t stride_w, int64_t pad_h,
                       int64_t pad_w, void* stream);

/* NCHW convolution with zero padding (conv2d/kernel.py:6-49); bias may be NULL. fp32 runs as
 * an implicit GEMM on MFMA (the input patches are gathered while staging, never
 * materialised); bf16/fp16 use a direct kernel. fp32 accumulation. */
int dli_hip_conv2d(int dtype, const void* x, const void* weight, const void* bias, void* out,
                   int64_t n, int64_t in_c, int64_t h, int64_t w, int64_t out_c,
                   int64_t kernel_h, int64_t kernel_w, int64_t out_h, int64_t out_w,
                   int64_t stride_h, int64_t stride_w, int64_t pad_h, int64_t pad_w,
                   void* stream);

/* dli_hip_conv2d followed by `activation` (DLI_ACT_*), fused into the GEMM epilogue on the
 * MFMA path. No counterpart in the reference, whose graph runs conv2d and relu as two nodes
 * (conv2d/kernel.py:6-49, relu/kernel.py:6); the plugin uses it for a conv2d node with
 * attribute activation = "relu". workspace as for dli_hip_linear_act (NULL: no split). */
int dli_hip_conv2d_act(int dtype, const void* x, const void* weight, const void* bias,
                       void* out, int64_t n, int64_t in_c, int64_t h, int64_t w, int64_t out_c,
                       int64_t kernel_h, int64_t kernel_w, int64_t out_h, int64_t out_w,
                       int64_t stride_h, int64_t stride_w, int64_t pad_h, int64_t pad_w,
                       int activation, void* workspace, size_t workspace_bytes, void* stream);
/* Workspace bytes that let dli_hip_conv2d_act split an fp32 conv's patch dimension over more
 * workgroups when its output tiles alone leave CUs idle (0: no split). No zeroing needed; the
 * splits are summed in a fixed order. */
size_t dli_hip_conv2d_workspace(int dtype, int64_t n, int64_t in_c, int64_t out_c,
                                int64_t kernel_h, int64_t kernel_w, int64_t out_h, int64_t out_w);

/* out[m, n] = sum_k x[m, k] * w[n, k] (+ bias[n]) (linear/kernel.py:6-44;
 * linear/template.cc:23-32). x, w, bias share `dtype`; out_dtype is dtype or DLI_F32.
 * bias may be NULL. fp32 accumulation. MFMA: fp32 always (16x16x4 f32); bf16 as a weight
 * stream for m <= 64 (K % 64 == 0), else as tiled bf16 MFMA (K % 8 == 0, 16-byte aligned). */
int dli_hip_linear(int dtype, int out_dtype, const void* x, const void* w, const void* bias,
                   void* out, int64_t m, int64_t n, int64_t k, void* stream);

/* dli_hip_linear followed by `activation` (DLI_ACT_*), fused into the epilogue on the tiled
 * MFMA paths. No counterpart in the reference (linear and relu are separate nodes there); the
 * plugin uses it for every linear node (attribute activation = "relu" to fuse). A workspace of
 * dli_hip_linear_workspace(dtype, m, n, k) bytes (no zeroing needed) lets fp32 shapes with few
 * output tiles and a long K, and bf16 shapes with 33-64 rows (or 9-32 rows and n >= 8192, which
 * run on the tiled GEMM) and few output tiles, split K over more workgroups, summing the splits
 * in a fixed order; with workspace NULL or smaller, fewer or no splits. */
int dli_hip_linear_act(int dtype, int out_dtype, const void* x, const void* w, const void* bias,
                       void* out, int64_t m, int64_t n, int64_t k, int activation,
                       void* workspace, size_t workspace_bytes, void* stream);
size_t dli_hip_linear_workspace(int dtype, int64_t m, int64_t n, int64_t k);

/* out[m, n] = sum_k a[m, k] * b[k, n] (matmul/kernel.py:6-40); fp32 on MFMA. */
int dli_hip_matmul(int dtype, const void* a, const void* b, void* out, int64_t m, int64_t n,
                   int64_t k, void* stream);

/* Interleaved-pair rotary embedding (rotary/kernel.py:6-35): for pair p of head-vector v at
 * token t, with c = cos[pos, p], s = sin[pos, p]:
 *   out[2p] = x[2p]*c - x[2p+1]*s ;  out[2p+1] = x[2p]*s + x[2p+1]*c
 * q is [batch, q_heads, seq, head_dim], k is [batch, k_heads, seq, head_dim]; cos/sin are fp32
 * [max_pos, pairs]; pairs <= head_dim/2 (dims beyond 2*pairs are copied). Position:
 * pos = start_pos + t, plus positions[b] when positions is non-NULL (int32/int64 [batch]).
 * Positions outside [0, max_pos) leave the pair unrotated. */
int dli_hip_rotary(int dtype, const void* q, const void* k, const float* cos_table,
                   const float* sin_table, void* out_q, void* out_k, int64_t batch,
                   int64_t q_heads, int64_t k_heads, int64_t seq, int64_t head_dim,
                   int64_t pairs, int64_t max_pos, int64_t start_pos, const void* positions,
                   int positions_dtype, void* stream);

/* Softmax attention over contiguous [B, H, S, D] tensors (attention/kernel.py:6-62), with
 * grouped KV heads (q head h reads kv head h / (q_heads / kv_heads)) and the causal rule
 * key <= (seq_k - seq_q) + query. scale is usually 1/sqrt(head_dim). head_dim <= 256.
 * bf16 with head_dim 64 and 16-byte aligned tensors (prefill) runs as a flash-style MFMA
 * kernel; other cases as one wave per query row. */
int dli_hip_attention(int dtype, const void* q, const void* k, const void* v, void* out,
                      int64_t batch, int64_t q_heads, int64_t kv_heads, int64_t seq_q,
                      int64_t seq_k, int64_t head_dim, int causal, float scale, void* stream);

/* dli_hip_attention with out as [batch, seq_q, q_heads, head_dim], written by the attention
 * kernel itself: the layout the merge reshape after attention (export.py:358-375) needs, which a
 * prompt's [B, H, S, D] output reaches only through a transpose node. No counterpart in the
 * reference (it fuses that transpose); the fused prefill graph uses it. Only the flash path
 * (bf16, head_dim 64, seq_k > 0, 16-byte aligned tensors): any other call is rejected
 * (DLI_HIP_EINVAL). */
int dli_hip_attention_bshd(int dtype, const void* q, const void* k, const void* v, void* out,
                           int64_t batch, int64_t q_heads, int64_t kv_heads, int64_t seq_q,
                           int64_t seq_k, int64_t head_dim, int causal, float scale,
                           void* stream);

/* Writes key/value [B, H, S, D] into the paged cache (layout in include/dli/kv_cache.h):
 * token s of sequence b goes to position p = start + s, or positions[b] + s when positions is
 * non-NULL. Tokens at p >= max_blocks * block_size are dropped. */
int dli_hip_kv_append(int dtype, const void* key, const void* value, void* key_pool,
                      void* value_pool, const int32_t* block_table, int64_t batch,
                      int64_t heads, int64_t seq, int64_t head_dim, int64_t block_size,
                      int64_t max_blocks, int64_t start, const void* positions,
                      int positions_dtype, void* stream);

/* Attention of q [B, Hq, Sq, D] over the paged cache. Sequence b holds
 * L_b = past_len + Sq tokens (past_len = positions[b] when positions is non-NULL, else
 * `past`); the query at index i sits at position past_len + i and, when causal, sees keys
 * at positions <= past_len + i. Split along the keys across workgroups ("flash decoding");
 * partial results and per-(sequence, kv head) arrival counters go to `workspace` (size from
 * dli_hip_paged_attention_workspace, the same offsets for every head_dim). The workspace must be
 * zero-filled before its first use; every call leaves the counters at zero again. Calls sharing
 * a workspace must be ordered (same stream). splits: the key-range split count of the MFMA
 * decode kernel (bf16, one query per sequence), 0 = about one workgroup per CU, else in [1, 32];
 * dli_hip_decoder_stack with the same attention_splits gives bit-identical results. */
size_t dli_hip_paged_attention_workspace(int64_t batch, int64_t q_heads, int64_t seq_q,
                                         int64_t head_dim, int64_t max_tokens);
int dli_hip_paged_attention(int dtype, const void* q, const void* key_pool,
                            const void* value_pool, const int32_t* block_table, void* out,
                            int64_t batch, int64_t q_heads, int64_t kv_heads, int64_t seq_q,
                            int64_t head_dim, int64_t block_size, int64_t max_blocks,
                            int64_t past, const void* positions, int positions_dtype,
                            int causal, float scale, int splits, void* workspace,
                            size_t workspace_bytes, void* stream);

/* ids[r] = first index of the maximum of row r of x [rows, width] (torch.argmax rule). */
int dli_hip_argmax(int dtype, const void* x, int64_t* ids, int64_t rows, int64_t width,
                   void* stream);

/* ---------------------------------------------------------------------------------------
 * 3. Fused bf16 decode kernels (batch rows m in [1, 64], reduction sizes multiple of 64,
 *    16-byte aligned x and weights). They replace runs of nodes of the reference's exported
 *    decoder graph (python/dli_export/export.py:272-446), keeping every node's bf16 rounding
 *    point. The RMSNorm in front of qkv and gate/up runs inside those kernels, on the
 *    activation fragments each workgroup loads (or, with dli_hip_linear_residual_norm, once
 *    after the residual update). Split-K variants use a caller workspace of
 *    dli_hip_splitk_workspace() bytes; calls that share one workspace must be ordered (same
 *    stream).
 * ------------------------------------------------------------------------------------- */

size_t dli_hip_splitk_workspace(int64_t n, int64_t m, int splits);

/* [xn = rms_norm(hidden) * norm_weight when norm_weight is non-NULL, else xn = hidden] ->
 * [q | k | v] = xn W_qkv^T + b -> interleaved RoPE on q and k at positions[b] -> k, v written
 * into the paged cache at positions[b] -> q_out [m, q_heads, head_dim]; hidden <= 1024.
 * W_qkv is [(q_heads + 2 kv_heads) * head_dim, hidden]; cos/sin are fp32 [max_pos,
 * head_dim / 2]. Replaces input_layernorm, q/k/v_proj, 3 reshapes, rotary_embedding and the
 * KV append inside attention (export.py:280-349; rotary/kernel.py:6-35). */
int dli_hip_qkv_rope_append(const void* hidden, const void* norm_weight, const void* w_qkv,
                            const void* b_qkv, const float* cos_table, const float* sin_table,
                            int64_t max_pos, const void* positions, int positions_dtype,
                            void* q_out, void* key_pool, void* value_pool,
                            const int32_t* block_table, int64_t block_size, int64_t max_blocks,
                            int64_t batch, int64_t hidden_size, int64_t q_heads, int64_t kv_heads,
                            int64_t head_dim, float eps, void* stream);

/* dli_hip_qkv_rope_append for any hidden size, with a caller workspace of
 * dli_hip_qkv_rope_append_workspace() bytes (0 when hidden <= 1024, where it is the call above).
 * Above 1024 (a large hidden size such as the Qwen2-7B geometry's 3584) norm_weight must be
 * NULL (the RMSNorm is a node of its own, or the previous dli_hip_linear_residual_norm), and the
 * projection runs as K-split fp32 parts in the workspace (the tiled MFMA GEMM from 33 rows, the
 * skinny kernels below) followed by one reduce that sums the parts in split order, adds the
 * bias, rotates q and k, writes q and puts k and v into the cache: the same values as the call
 * above and as the reference's q/k/v_proj, rotary_embedding and attention KV-append nodes
 * (export.py:280-349; rotary/kernel.py:6-35). Calls sharing a workspace must be ordered. */
size_t dli_hip_qkv_rope_append_workspace(int64_t batch, int64_t hidden_size, int64_t q_heads,
                                         int64_t kv_heads, int64_t head_dim);
int dli_hip_qkv_rope_append_ws(const void* hidden, const void* norm_weight, const void* w_qkv,
                               const void* b_qkv, const float* cos_table, const float* sin_table,
                               int64_t max_pos, const void* positions, int positions_dtype,
                               void* q_out, void* key_pool, void* value_pool,
                               const int32_t* block_table, int64_t block_size,
                               int64_t max_blocks, int64_t batch, int64_t hidden_size,
                               int64_t q_heads, int64_t kv_heads, int64_t head_dim, float eps,
                               void* workspace, size_t workspace_bytes, void* stream);

/* out = residual + (x W^T + b), the linear output rounded before the add. Replaces o_proj +
 * attention_residual and down_proj + mlp_residual (export.py:366-376, 416-424). splits in
 * [2, min(8, k / 64)] splits K over workgroups: each stores a partial tile in the workspace and
 * the last to finish a tile sums them in split order and writes it. The workspace
 * (dli_hip_splitk_workspace bytes) must be zero-filled before its first use; every call leaves
 * its arrival counters at zero again. With m > 64 (a prompt: k % 8 == 0) one tiled MFMA GEMM
 * computes it with the add in its epilogue; splits and the workspace are then not used. With
 * 9-64 rows and n > 1024 (outputs wider than the fused decode kernels hold, 33+ rows or
 * n >= 8192) the tiled GEMM splits K into fp32 parts in the workspace, as many as the workspace
 * of `splits` holds (up to its own choice), summed in split order with the residual by a second
 * kernel. */
int dli_hip_linear_residual(const void* x, const void* w, const void* bias, const void* residual,
                            void* out, int64_t m, int64_t n, int64_t k, int splits,
                            void* workspace, size_t workspace_bytes, void* stream);

/* h_out = residual + (x W^T + b) as above, and xn_out = rms_norm(h_out) * norm_weight, both
 * [m, n]. Replaces o_proj + attention_residual + post_attention_layernorm, and down_proj +
 * mlp_residual + the next layer's input_layernorm (or model.norm after the last layer)
 * (export.py:366-424; rms_norm/kernel.py:6-14). Always uses the workspace; splits in
 * [1, min(8, k / 64)]. n <= 1024: the fused residual kernels. 1024 < n <= 4096 (n % 8 == 0; a
 * large hidden size): K-split fp32 parts (the tiled MFMA GEMM from 33 rows, splitting K as far as
 * the workspace of `splits` holds, up to its own choice; the skinny kernels with `splits` parts
 * below), then one workgroup per row sums them in split order with the bias and the residual and
 * normalizes; residual, bias, norm_weight and both outputs 16-byte aligned. */
int dli_hip_linear_residual_norm(const void* x, const void* w, const void* bias,
                                 const void* residual, const void* norm_weight, void* h_out,
                                 void* xn_out, int64_t m, int64_t n, int64_t k, float eps,
                                 int splits, void* workspace, size_t workspace_bytes,
                                 void* stream);

/* [xn = rms_norm(hidden) * norm_weight when norm_weight is non-NULL, else xn = hidden] ->
 * gate/up projections of xn -> silu(gate) * up, out [m, ffn]; hidden <= 1024. w_gate_up
 * interleaves the two weights in blocks of 16 rows: rows [32i, 32i+16) = gate rows
 * [16i, 16i+16), rows [32i+16, 32i+32) = up rows [16i, 16i+16). Replaces
 * post_attention_layernorm, gate_proj, up_proj, act_fn and mul (export.py:378-414). With
 * m > 64 (a prompt), and at any m with hidden_size > 1024, one tiled MFMA GEMM over the
 * interleaved weight computes it, the SwiGLU in its epilogue (any hidden_size % 8 == 0);
 * norm_weight must then be NULL (normalize first). */
int dli_hip_gate_up_silu(const void* hidden, const void* norm_weight, const void* w_gate_up,
                         void* out, int64_t m, int64_t ffn, int64_t hidden_size, float eps,
                         void* stream);

/* Prefill form of the attention inputs: [q | k | v] = x W_qkv^T + b over the B * S tokens of a
 * prompt (x [batch, seq, hidden_size] bf16, normalized), each value rounded to bf16 as the
 * linear node rounds it; interleaved RoPE on q and k at position start_pos + s (cos/sin fp32
 * [max_pos, head_dim / 2]; positions outside the table unchanged), rounded as the rotary node
 * rounds it; q_out [batch, q_heads, seq, head_dim], k_out and v_out [batch, kv_heads, seq,
 * head_dim]. One tiled MFMA GEMM with the RoPE and the head layout in its epilogue. Replaces
 * q/k/v_proj, the three reshapes, the three [B,S,H,D] -> [B,H,S,D] transposes and
 * rotary_embedding of a prompt layer (export.py:280-349; rotary/kernel.py:6-35). head_dim % 8
 * == 0, hidden_size % 8 == 0, pointers (except cos/sin) 16-byte aligned. */
int dli_hip_qkv_rope_heads(const void* x, const void* w_qkv, const void* b_qkv, const float* cos,
                           const float* sin, int64_t max_pos, void* q_out, void* k_out,
                           void* v_out, int64_t batch, int64_t seq, int64_t hidden_size,
                           int64_t q_heads, int64_t kv_heads, int64_t head_dim, int64_t start_pos,
                           void* stream);

/* logits = xn W^T (fp32 accumulation) -> ids[m] = argmax (first maximum); hidden <= 1024.
 * logits may be NULL (only ids) or float32 / bfloat16 [m, vocab]. Replaces lm_head
 * (export.py:426-443) plus the greedy token choice. */
size_t dli_hip_lm_head_argmax_workspace(int64_t m, int64_t vocab);
int dli_hip_lm_head_argmax(const void* xn, const void* w, void* logits, int logits_dtype,
                           int64_t* ids, int64_t m, int64_t vocab, int64_t hidden_size,
                           void* workspace, size_t workspace_bytes, void* stream);
/* dli_hip_lm_head_argmax of the final RMSNorm of x: xn = bf16(x * rsqrt(mean(x^2) + eps) *
 * norm_weight) is computed in registers by every workgroup (rms_norm/kernel.py:6-14), so the
 * model.norm node needs no launch of its own. norm_weight [hidden] may be NULL (x is already
 * normalized). No counterpart in the reference, where model.norm and lm_head are two nodes
 * (export.py:420-443). */
int dli_hip_lm_head_argmax_norm(const void* x, const void* norm_weight, float eps, const void* w,
                                void* logits, int logits_dtype, int64_t* ids, int64_t m,
                                int64_t vocab, int64_t hidden_size, void* workspace,
                                size_t workspace_bytes, void* stream);
/* dli_hip_lm_head_argmax_norm without a workspace argument and without allocating: the argmax
 * partials (one per row and lm_head workgroup) go to a static 4 MiB device array of the library (one per device, set up on
 * the first call on that device, which also loads the kernels there; held until the process
 * ends). No counterpart in the reference: it is for callers that cannot allocate device memory
 * (code under HIP graph capture, tight serving loops, harnesses that forbid hipMalloc). Same
 * kernels and results as dli_hip_lm_head_argmax_norm; rejects (DLI_HIP_EINVAL) a call whose
 * partials, 8 * m * ceil(vocab / 32) bytes, exceed 4 MiB. Every call on a device shares that
 * array, so calls that overlap on one device (other streams, other threads) race. */
int dli_hip_lm_head_argmax_norm_noalloc(const void* x, const void* norm_weight, float eps,
                                        const void* w, void* logits, int logits_dtype,
                                        int64_t* ids, int64_t m, int64_t vocab,
                                        int64_t hidden_size, void* stream);

/* ---------------------------------------------------------------------------------------
 * 4. Persistent decoder stack: all decoder layers of one batched decode step in one launch
 *    (one 8-wave workgroup per CU). Per layer it computes exactly what the five fused calls
 *    above compute (dli_hip_qkv_rope_append with the input norm, dli_hip_paged_attention,
 *    dli_hip_linear_residual for o_proj with one split, dli_hip_gate_up_silu with the
 *    post-attention norm, dli_hip_linear_residual for down_proj with down_splits), bit for bit,
 *    and replaces the same reference nodes: export.py:272-424 for every layer. Workgroups hand
 *    stages to each other through arrival counters in the workspace instead of kernel
 *    boundaries. Supported: bf16, head_dim 64, block_size 64, q_heads / kv_heads <= 16,
 *    hidden <= 1024 and a multiple of 64, ffn a multiple of 64, batch <= 64, no o_proj or
 *    down_proj bias.
 * ------------------------------------------------------------------------------------- */

/* Device pointers of one decoder layer. */
typedef struct DliDecoderLayer {
  const void* input_norm;      /* [hidden] */
  const void* w_qkv;           /* [(q_heads + 2 kv_heads) head_dim, hidden], rows q | k | v */
  const void* b_qkv;           /* [(q_heads + 2 kv_heads) head_dim] or NULL */
  const void* w_o;             /* [hidden, q_heads head_dim] */
  const void* post_norm;       /* [hidden] */
  const void* w_gate_up;       /* [2 ffn, hidden], 16-row interleave as dli_hip_gate_up_silu */
  const void* w_down;          /* [hidden, ffn] */
  void* key_pool;              /* paged cache of this layer (include/dli/kv_cache.h) */
  void* value_pool;
  const int32_t* block_table;  /* [batch, max_blocks] */
} DliDecoderLayer;

/* Per-call options of dli_hip_decoder_stack (NULL = all zero).
 * attention_splits: key-range splits per (sequence, kv head) attention pair, 0 = spread the
 *   pairs over the CUs the q|k|v stage leaves free, else in [1, 32] (the same count as
 *   dli_hip_paged_attention's splits gives bit-identical results).
 * trace, trace_layers: stage timeline (no counterpart in the reference; its profiler exists only
 *   as a design, .codex/profiling_design.md). With trace non-NULL the launch stamps the 100 MHz
 *   real-time counter (s_memrealtime) at the stage boundaries of each workgroup:
 *   trace[(layer * grid + workgroup) * DLI_STACK_TRACE_EVENTS + event] for layer < trace_layers,
 *   where grid is the
 *   launch's workgroup count (one per CU) and the events are those of dli_stack::kTr* in
 *   csrc/kernels/stack_args.h (0 = layer entry ... 12 = down_proj done). The buffer holds
 *   trace_layers * grid * DLI_STACK_TRACE_EVENTS uint64 of device memory; events a workgroup
 *   does not reach are left
 *   as they were.
 * token_ids, token_ids_dtype, embedding, vocab: with token_ids non-NULL (device [batch],
 *   token_ids_dtype DLI_I64 or DLI_I32) the first layer's input is row token_ids[b] of
 *   embedding (device bf16 [vocab, hidden_size], 16-byte aligned; a zero row for an id outside
 *   [0, vocab)), which is what dli_hip_embedding writes, gathered by the launch itself, and
 *   hidden_in is not read (it may be NULL). This folds the model.embed_tokens node
 *   (export.py:273-279) into the launch and saves its kernel launch per step. */
#define DLI_STACK_TRACE_EVENTS 32
typedef struct DliStackOptions {
  int attention_splits;
  unsigned long long* trace;
  int trace_layers;
  const void* token_ids;
  int token_ids_dtype;
  const void* embedding;
  int64_t vocab;
} DliStackOptions;

/* Workspace bytes for dli_hip_decoder_stack with num_layers layers (arrival counters, partials
 * and one activation slab per layer of a launch, so no activation buffer is reused within a
 * launch), for the given down_splits and attention_splits (0 = the launch's own choice). */
size_t dli_hip_decoder_stack_workspace(int num_layers, int64_t batch, int64_t hidden_size,
                                       int64_t q_heads, int64_t kv_heads, int64_t head_dim,
                                       int64_t ffn, int64_t max_blocks, int down_splits,
                                       int attention_splits);

/* hidden_out = the residual stream after `num_layers` layers applied to hidden_in [batch,
 * hidden_size] (hidden_out may equal hidden_in; or to the embedding rows of options->token_ids). Each layer appends its new k/v at
 * positions[b] and attends over keys [0, positions[b]]. The workspace must be zero-filled
 * before its first use; every call leaves it ready for the next one on the same stream. Calls
 * that share a workspace must not overlap.
 * The launch is refused when the device cannot hold every workgroup resident at once; it is a
 * plain kernel launch (or graph node), so work running on other streams at the same time can hold
 * workgroups back and make a wait give up (reported through status). status (device memory, may be NULL): when
 * non-NULL, a launch in which a wait gave up ORs a non-zero value into *status and clears the
 * workspace's abort word, so later launches run normally; the caller reads *status after a
 * synchronization it already makes and zeroes it. With status NULL the abort word stays set for
 * dli_hip_decoder_stack_status. */
int dli_hip_decoder_stack(const DliDecoderLayer* layers, int num_layers, const void* hidden_in,
                          void* hidden_out, const void* positions, int positions_dtype,
                          const float* cos_table, const float* sin_table, int64_t max_pos,
                          int64_t block_size, int64_t max_blocks, int64_t batch,
                          int64_t hidden_size, int64_t q_heads, int64_t kv_heads,
                          int64_t head_dim, int64_t ffn, float eps, int down_splits,
                          void* workspace, size_t workspace_bytes, unsigned* status,
                          const DliStackOptions* options, void* stream);

/* Synchronizes `stream`, then *aborted = 1 when a launch since the last query gave up waiting
 * for another workgroup (its outputs are invalid; this can only happen when the workgroups
 * were not all resident at once), else 0. Clears the flag. */
int dli_hip_decoder_stack_status(void* workspace, int* aborted, void* stream);

#ifdef __cplusplus
}  /* extern "C" */
#endif

#endif  /* DLI_HIP_H_ */
