#pragma once

// Shared device helpers for the gfx950 kernels of libdli_hip.so.
// Storage types: float, bf16 (raw 16-bit, converted with round-to-nearest-even, NaN kept
// quiet) and _Float16. All arithmetic is fp32.

#include <hip/hip_runtime.h>
#include <stdint.h>

namespace dk {

constexpr int kWave = 64;

// First statement of a function whose floating-point results must not depend on where it is
// inlined: no multiply-add contraction, so every kernel that shares the function rounds
// identically (the fused and the persistent decode paths are compared bit for bit).
#define FP_EXACT _Pragma("clang fp contract(off)")

// A wait that is not needed (data produced by an earlier launch).
struct NoWait {
  __device__ __forceinline__ void operator()() const {}
};

// Global-memory view of a pointer into device memory. Accesses through it compile to global_*
// instructions; through a generic pointer whose origin the compiler cannot trace (a pointer that
// passed through an asm statement, a select, a struct) they become flat_* instructions, which
// also count against lgkmcnt and so merge their waits with those of LDS operations.
#define DK_GLOBAL __attribute__((address_space(1)))
template <typename T>
__device__ __forceinline__ DK_GLOBAL T* gp(T* p) {
  return (DK_GLOBAL T*)p;
}
template <typename T>
__device__ __forceinline__ const DK_GLOBAL T* gp(const T* p) {
  return (const DK_GLOBAL T*)p;
}

// Tagged words: an fp32 value and a 32-bit tag in one 8-byte word, written with one agent-scope
// (single-copy atomic) store. A reader that sees the tag it expects has the value that came with
// it, without a counter or a store acknowledgement in between. For hand-offs between workgroups
// that are all resident at once (a persistent launch), each word written by one workgroup per
// tag value.
constexpr int kTagSpinLimit = 1 << 20;

__device__ __forceinline__ void storeTaggedBits(uint64_t* p, uint32_t bits, unsigned tag) {
  __hip_atomic_store(gp(p), (static_cast<uint64_t>(tag) << 32) | bits, __ATOMIC_RELAXED,
                     __HIP_MEMORY_SCOPE_AGENT);
}

__device__ __forceinline__ void storeTagged(uint64_t* p, float v, unsigned tag) {
  storeTaggedBits(p, __float_as_uint(v), tag);
}

__device__ __forceinline__ void fromBits(float& v, uint32_t bits) { v = __uint_as_float(bits); }
__device__ __forceinline__ void fromBits(uint32_t& v, uint32_t bits) { v = bits; }

// v[i] = the value at p[i] once its tag is `tag`, for i < n (all n loads in flight at once, the
// set reread until every tag matches). Gives up after kTagSpinLimit rounds, or once *abort_word
// is non-zero, and then sets *abort_word (the values are then invalid). T: float, or uint32_t
// for the raw 32 bits (two packed bf16).
template <int N, class T>
__device__ __forceinline__ void loadTagged(T (&v)[N], const uint64_t* const (&p)[N], int n,
                                           unsigned tag, unsigned* abort_word) {
  for (int spins = 0;; ++spins) {
    uint64_t w[N];
#pragma unroll
    for (int i = 0; i < N; ++i)
      w[i] = i < n ? __hip_atomic_load(gp(p[i]), __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT)
                   : static_cast<uint64_t>(tag) << 32;
    bool ok = true;
#pragma unroll
    for (int i = 0; i < N; ++i) {
      ok = ok && static_cast<unsigned>(w[i] >> 32) == tag;
      fromBits(v[i], static_cast<uint32_t>(w[i]));
    }
    if (ok) return;
    if (spins >= kTagSpinLimit ||
        (spins % 64 == 63 &&
         __hip_atomic_load(gp(abort_word), __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT) != 0u)) {
      __hip_atomic_store(gp(abort_word), 1u, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
      return;
    }
    __builtin_amdgcn_s_sleep(1);
  }
}

// Timeline hook of a stage helper: mark(point) at its internal points (a no-op by default).
struct NoMark {
  __device__ __forceinline__ void operator()(int) const {}
};

// threadIdx.x passed through an empty asm statement. Per-lane offsets computed from it are then
// recomputed where a long kernel uses them, instead of being computed once at the start and
// held in registers (or spilled to scratch) across everything in between.
__device__ __forceinline__ int freshThreadIdx() {
  int t = static_cast<int>(threadIdx.x);
  asm volatile("" : "+v"(t));
  return t;
}

struct bf16 {
  uint16_t bits;
};
using f16 = _Float16;

__device__ __forceinline__ float bf16ToFloat(uint16_t bits) {
  return __uint_as_float(static_cast<uint32_t>(bits) << 16);
}

// Round-to-nearest-even, the rule torch uses for float -> bfloat16 (gfx950 converts in hardware:
// v_cvt_pk_bf16_f32; NaN stays NaN).
__device__ __forceinline__ uint16_t floatToBf16(float f) {
  return __builtin_bit_cast(uint16_t, static_cast<__bf16>(f));
}

typedef float f32x2_t __attribute__((ext_vector_type(2)));
typedef __bf16 bf16x2_t __attribute__((ext_vector_type(2)));

// Two floats -> two bfloat16 (RNE) packed as lo | hi << 16, one conversion instruction.
__device__ __forceinline__ uint32_t packBf16x2(float lo, float hi) {
  return __builtin_bit_cast(uint32_t, __builtin_convertvector(f32x2_t{lo, hi}, bf16x2_t));
}

template <typename T>
struct Num;

template <>
struct Num<float> {
  static __device__ __forceinline__ float load(const float* p) { return *p; }
  static __device__ __forceinline__ void store(float* p, float v) { *p = v; }
  static __device__ __forceinline__ float round(float v) { return v; }
};

template <>
struct Num<bf16> {
  static __device__ __forceinline__ float load(const bf16* p) { return bf16ToFloat(p->bits); }
  static __device__ __forceinline__ void store(bf16* p, float v) { p->bits = floatToBf16(v); }
  static __device__ __forceinline__ float round(float v) { return bf16ToFloat(floatToBf16(v)); }
};

template <>
struct Num<f16> {
  static __device__ __forceinline__ float load(const f16* p) { return static_cast<float>(*p); }
  static __device__ __forceinline__ void store(f16* p, float v) { *p = static_cast<f16>(v); }
  static __device__ __forceinline__ float round(float v) {
    return static_cast<float>(static_cast<f16>(v));
  }
};

template <typename T>
__device__ __forceinline__ float ld(const T* p) {
  return Num<T>::load(p);
}
template <typename T>
__device__ __forceinline__ void st(T* p, float v) {
  Num<T>::store(p, v);
}

// Reductions over the four 16-lane rows of a wave (lanes l, l ^ 16, l ^ 32, l ^ 48) with the
// gfx950 permlane swaps (VALU, no LDS round trip). permlaneNN_swap(x, x) yields, in every lane,
// {x[l & ~NN], x[l | NN]}; every lane then combines the same two operands in the same order,
// and since IEEE addition and fmax are commutative the results equal the xor-shuffle forms
// v op v[l ^ 16], then op v[l ^ 32], bit for bit.
__device__ __forceinline__ float rowsSum(float v) {
  const auto a = __builtin_amdgcn_permlane16_swap(__float_as_uint(v), __float_as_uint(v), false,
                                                  false);
  v = __uint_as_float(a[0]) + __uint_as_float(a[1]);
  const auto b = __builtin_amdgcn_permlane32_swap(__float_as_uint(v), __float_as_uint(v), false,
                                                  false);
  return __uint_as_float(b[0]) + __uint_as_float(b[1]);
}

__device__ __forceinline__ float rowsMax(float v) {
  const auto a = __builtin_amdgcn_permlane16_swap(__float_as_uint(v), __float_as_uint(v), false,
                                                  false);
  v = fmaxf(__uint_as_float(a[0]), __uint_as_float(a[1]));
  const auto b = __builtin_amdgcn_permlane32_swap(__float_as_uint(v), __float_as_uint(v), false,
                                                  false);
  return fmaxf(__uint_as_float(b[0]), __uint_as_float(b[1]));
}

__device__ __forceinline__ float waveSum(float v) {
#pragma unroll
  for (int offset = kWave / 2; offset > 0; offset >>= 1) v += __shfl_xor(v, offset, kWave);
  return v;
}

__device__ __forceinline__ float waveMax(float v) {
#pragma unroll
  for (int offset = kWave / 2; offset > 0; offset >>= 1) v = fmaxf(v, __shfl_xor(v, offset, kWave));
  return v;
}

// Sum over the whole block; `scratch` holds one float per wave. Every thread gets the result.
__device__ __forceinline__ float blockSum(float v, float* scratch) {
  const int lane = threadIdx.x % kWave;
  const int wave = threadIdx.x / kWave;
  const int waves = (blockDim.x + kWave - 1) / kWave;
  v = waveSum(v);
  __syncthreads();
  if (lane == 0) scratch[wave] = v;
  __syncthreads();
  float total = 0.f;
  for (int w = 0; w < waves; ++w) total += scratch[w];
  return total;
}

__device__ __forceinline__ float blockMax(float v, float* scratch) {
  const int lane = threadIdx.x % kWave;
  const int wave = threadIdx.x / kWave;
  const int waves = (blockDim.x + kWave - 1) / kWave;
  v = waveMax(v);
  __syncthreads();
  if (lane == 0) scratch[wave] = v;
  __syncthreads();
  float m = -INFINITY;
  for (int w = 0; w < waves; ++w) m = fmaxf(m, scratch[w]);
  return m;
}

__device__ __forceinline__ int64_t loadIndex(const void* p, int is64, int64_t i) {
  return is64 ? gp(static_cast<const int64_t*>(p))[i]
              : static_cast<int64_t>(gp(static_cast<const int32_t*>(p))[i]);
}

}  // namespace dk

// Instantiates `extern "C"` kernels named <base>_f32 / _bf16 / _f16 from a template kernel body
// `base##_impl<T>`; ARGS/CALL are the parameter list and the forwarding argument list.
#define DK_FLOAT_KERNELS(base, bounds, ARGS, CALL)                                        \
  extern "C" __global__ void __launch_bounds__(bounds) base##_f32 ARGS {                  \
    base##_impl<float> CALL;                                                              \
  }                                                                                       \
  extern "C" __global__ void __launch_bounds__(bounds) base##_bf16 ARGS {                 \
    base##_impl<dk::bf16> CALL;                                                           \
  }                                                                                       \
  extern "C" __global__ void __launch_bounds__(bounds) base##_f16 ARGS {                  \
    base##_impl<dk::f16> CALL;                                                            \
  }
