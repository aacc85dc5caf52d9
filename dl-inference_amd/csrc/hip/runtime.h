#pragma once

// Internal C++ side of libdli_hip.so: the dlopen'd HIP runtime table, error reporting, and
// lazily loaded per-device kernels from the embedded gfx950 code objects.

#include <array>
#include <atomic>
#include <cstddef>
#include <cstdint>
#include <mutex>
#include <string>

#include "dli_hip.h"

namespace dli::hip {

struct Dim3 {
  unsigned x = 1, y = 1, z = 1;
};

// Records `message` as this thread's last error and returns `code`.
int fail(int code, const std::string& message);
// Maps a hipError_t to 0 / a recorded error with context.
int check(int hip_status, const char* what);
int requireRuntime();
// Compute units of the current device (cached per device).
int computeUnits(int* count);
// Key-range splits per workgroup unit of MFMA decode attention (a (sequence, kv head) pair, or a
// group of kv heads of one sequence): about `cus` workgroups over all units, no more splits than
// groups of wph cache blocks (wph: waves per kv head); `requested` > 0 (the caller's count)
// replaces the per-CU choice. Never fewer splits than the per-lane block ids of a wave allow.
int decodeAttentionSplits(int64_t units, int64_t max_blocks, int cus, int wph, int requested);
constexpr int kMaxDecodeSplits = 32;  // key-range splits a decode-attention call may use

// A kernel by name inside one embedded code object; resolved once per device.
class DeviceKernel {
 public:
  DeviceKernel(const char* module, const char* name) : module_(module), name_(name) {}
  // Returns 0 and the function handle for the current device, or an error code.
  int resolve(void** function);
  const char* name() const { return name_; }

 private:
  static constexpr int kMaxDevices = 64;
  const char* module_;
  const char* name_;
  std::array<std::atomic<void*>, kMaxDevices> functions_{};
  std::mutex mutex_;
};

int launchRaw(DeviceKernel& kernel, Dim3 grid, Dim3 block, unsigned lds_bytes, void* stream,
              void** args);

// launchRaw for a kernel whose workgroups wait on each other (a persistent launch): refuses a
// grid larger than the device can hold resident at once (occupancy query against the compute
// unit count), then launches it as a plain kernel (a plain kernel node under stream capture).
int launchResidentRaw(DeviceKernel& kernel, Dim3 grid, Dim3 block, unsigned lds_bytes,
                      void* stream, void** args);

// Device address and size of the global variable `name` of embedded code object `module`, for
// the current device (the module is loaded on that device first). hipModuleGetGlobal is the
// module-API lookup of a __device__ variable: each device that loads the module holds its own
// copy at its own address.
int moduleGlobal(const char* module, const char* name, void** ptr, size_t* bytes);

template <typename... Args>
int launchResident(DeviceKernel& kernel, Dim3 grid, Dim3 block, unsigned lds_bytes,
                   void* stream, Args... args) {
  if (grid.x == 0 || grid.y == 0 || grid.z == 0) return 0;
  void* params[] = {static_cast<void*>(&args)..., nullptr};
  return launchResidentRaw(kernel, grid, block, lds_bytes, stream, params);
}

template <typename... Args>
int launch(DeviceKernel& kernel, Dim3 grid, Dim3 block, unsigned lds_bytes, void* stream,
           Args... args) {
  if (grid.x == 0 || grid.y == 0 || grid.z == 0) return 0;
  void* params[] = {static_cast<void*>(&args)..., nullptr};
  return launchRaw(kernel, grid, block, lds_bytes, stream, params);
}

inline unsigned blocksFor(int64_t work, int64_t per_block) {
  return static_cast<unsigned>((work + per_block - 1) / per_block);
}

}  // namespace dli::hip
