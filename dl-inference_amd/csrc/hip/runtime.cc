// HIP module-load / launch / allocator layer of libdli_hip.so.
//
// Replaces src/cuda_driver.cc and src/cuda_runtime.cc of the reference (which dlopen libcuda /
// libcudart). The HIP runtime is dlopen'd the same way, so the library loads on machines
// without a GPU and reports why it cannot run. When PyTorch has already loaded its own copy of
// libamdhip64 (same soname), dlopen returns that copy, so torch and these kernels share one
// runtime, one device context and the same streams.
#include "runtime.h"

#include <dlfcn.h>

#include <cstring>
#include <map>
#include <utility>
#include <vector>

namespace dli::hip {
namespace {

using Status = int;  // hipError_t
using ModuleT = void*;
using FunctionT = void*;
using StreamT = void*;
using EventT = void*;

struct Runtime {
  void* handle = nullptr;
  std::string load_error;
  int device_count = 0;

  Status (*getDeviceCount)(int*) = nullptr;
  Status (*getDevice)(int*) = nullptr;
  Status (*setDevice)(int) = nullptr;
  Status (*moduleLoadData)(ModuleT*, const void*) = nullptr;
  Status (*moduleGetFunction)(FunctionT*, ModuleT, const char*) = nullptr;
  Status (*moduleUnload)(ModuleT) = nullptr;
  Status (*moduleLaunchKernel)(FunctionT, unsigned, unsigned, unsigned, unsigned, unsigned,
                               unsigned, unsigned, StreamT, void**, void**) = nullptr;
  Status (*malloc_)(void**, size_t) = nullptr;
  Status (*free_)(void*) = nullptr;
  Status (*memcpy_)(void*, const void*, size_t, int) = nullptr;
  Status (*memcpyAsync)(void*, const void*, size_t, int, StreamT) = nullptr;
  Status (*streamSynchronize)(StreamT) = nullptr;
  Status (*deviceSynchronize)() = nullptr;
  const char* (*getErrorString)(Status) = nullptr;
  Status (*eventCreate)(EventT*) = nullptr;
  Status (*eventRecord)(EventT, StreamT) = nullptr;
  Status (*eventSynchronize)(EventT) = nullptr;
  Status (*eventElapsedTime)(float*, EventT, EventT) = nullptr;
  Status (*eventDestroy)(EventT) = nullptr;
  Status (*deviceGetAttribute)(int*, int, int) = nullptr;
  Status (*streamIsCapturing)(StreamT, int*) = nullptr;
  Status (*moduleGetGlobal)(void**, size_t*, ModuleT, const char*) = nullptr;
  Status (*moduleOccupancy)(int*, FunctionT, int, size_t) = nullptr;

  template <typename F>
  bool bind(F& slot, const char* symbol) {
    slot = reinterpret_cast<F>(dlsym(handle, symbol));
    if (slot == nullptr) load_error = std::string("HIP runtime is missing symbol ") + symbol;
    return slot != nullptr;
  }

  Runtime() {
    const char* candidates[] = {"libamdhip64.so.7", "libamdhip64.so", "libamdhip64.so.6"};
    for (const char* name : candidates) {
      handle = dlopen(name, RTLD_NOW | RTLD_GLOBAL);
      if (handle != nullptr) break;
      if (const char* why = dlerror()) load_error = why;
    }
    if (handle == nullptr) {
      if (load_error.empty()) load_error = "libamdhip64 not found";
      return;
    }
    const bool ok = bind(getDeviceCount, "hipGetDeviceCount") && bind(getDevice, "hipGetDevice") &&
                    bind(setDevice, "hipSetDevice") &&
                    bind(moduleLoadData, "hipModuleLoadData") &&
                    bind(moduleGetFunction, "hipModuleGetFunction") &&
                    bind(moduleUnload, "hipModuleUnload") &&
                    bind(moduleLaunchKernel, "hipModuleLaunchKernel") &&
                    bind(malloc_, "hipMalloc") && bind(free_, "hipFree") &&
                    bind(memcpy_, "hipMemcpy") && bind(memcpyAsync, "hipMemcpyAsync") &&
                    bind(streamSynchronize, "hipStreamSynchronize") &&
                    bind(deviceSynchronize, "hipDeviceSynchronize") &&
                    bind(getErrorString, "hipGetErrorString") &&
                    bind(eventCreate, "hipEventCreate") && bind(eventRecord, "hipEventRecord") &&
                    bind(eventSynchronize, "hipEventSynchronize") &&
                    bind(eventElapsedTime, "hipEventElapsedTime") &&
                    bind(eventDestroy, "hipEventDestroy") &&
                    bind(deviceGetAttribute, "hipDeviceGetAttribute") &&
                    bind(streamIsCapturing, "hipStreamIsCapturing") &&
                    bind(moduleGetGlobal, "hipModuleGetGlobal") &&
                    bind(moduleOccupancy, "hipModuleOccupancyMaxActiveBlocksPerMultiprocessor");
    if (!ok) {
      dlclose(handle);
      handle = nullptr;
      return;
    }
    const Status status = getDeviceCount(&device_count);
    if (status != 0 || device_count <= 0) {
      load_error = std::string("no HIP device available: ") +
                   (status != 0 ? getErrorString(status) : "device count is 0");
      device_count = 0;
    } else {
      load_error.clear();
    }
  }
};

Runtime& runtime() {
  static Runtime* instance = new Runtime;  // intentionally leaked: valid during static teardown
  return *instance;
}

thread_local std::string t_last_error;

// Embedded code objects (generated at build time: symbols dli_co_<name> / dli_co_<name>_end).
struct CodeObject {
  const char* name;
  const unsigned char* begin;
  const unsigned char* end;
};

}  // namespace
}  // namespace dli::hip

#include "code_objects.inc"  // defines dli::hip::kCodeObjects[] and DLI_HIP_TARGET_ARCH

namespace dli::hip {
namespace {

struct ModuleCache {
  std::mutex mutex;
  std::map<std::pair<int, std::string>, ModuleT> modules;
};

ModuleCache& moduleCache() {
  static ModuleCache* cache = new ModuleCache;
  return *cache;
}

int loadEmbeddedModule(int device, const char* name, ModuleT* module) {
  auto& cache = moduleCache();
  std::lock_guard<std::mutex> lock(cache.mutex);
  auto key = std::make_pair(device, std::string(name));
  auto it = cache.modules.find(key);
  if (it != cache.modules.end()) {
    *module = it->second;
    return 0;
  }
  for (const CodeObject& co : kCodeObjects) {
    if (std::strcmp(co.name, name) != 0) continue;
    if (co.end <= co.begin) return fail(DLI_HIP_ENODEV, std::string("empty code object: ") + name);
    ModuleT loaded = nullptr;
    if (int rc = check(runtime().moduleLoadData(&loaded, co.begin), "hipModuleLoadData")) return rc;
    cache.modules.emplace(key, loaded);
    *module = loaded;
    return 0;
  }
  return fail(DLI_HIP_EINVAL, std::string("no embedded code object named ") + name);
}

}  // namespace

int fail(int code, const std::string& message) {
  t_last_error = message;
  return code;
}

int check(int hip_status, const char* what) {
  if (hip_status == 0) return 0;
  const char* text = runtime().getErrorString ? runtime().getErrorString(hip_status) : "unknown";
  return fail(hip_status, std::string(what) + " failed: " + (text ? text : "unknown"));
}

int requireRuntime() {
  Runtime& rt = runtime();
  if (rt.handle == nullptr || rt.device_count <= 0)
    return fail(DLI_HIP_ENODEV, "HIP runtime is unavailable: " + rt.load_error);
  return 0;
}

int computeUnits(int* count) {
  constexpr int kMultiprocessorCount = 63;  // hipDeviceAttributeMultiprocessorCount
  static std::array<std::atomic<int>, 64> cached{};
  if (int rc = requireRuntime()) return rc;
  int device = 0;
  if (int rc = check(runtime().getDevice(&device), "hipGetDevice")) return rc;
  if (device < 0 || device >= 64) return fail(DLI_HIP_EINVAL, "device index out of range");
  int value = cached[device].load(std::memory_order_relaxed);
  if (value <= 0) {
    if (int rc = check(runtime().deviceGetAttribute(&value, kMultiprocessorCount, device),
                       "hipDeviceGetAttribute"))
      return rc;
    cached[device].store(value, std::memory_order_relaxed);
  }
  *count = value;
  return 0;
}

int DeviceKernel::resolve(void** function) {
  if (int rc = requireRuntime()) return rc;
  int device = 0;
  if (int rc = check(runtime().getDevice(&device), "hipGetDevice")) return rc;
  if (device < 0 || device >= kMaxDevices) return fail(DLI_HIP_EINVAL, "device index out of range");
  void* cached = functions_[device].load(std::memory_order_acquire);
  if (cached != nullptr) {
    *function = cached;
    return 0;
  }
  std::lock_guard<std::mutex> lock(mutex_);
  cached = functions_[device].load(std::memory_order_relaxed);
  if (cached == nullptr) {
    ModuleT module = nullptr;
    if (int rc = loadEmbeddedModule(device, module_, &module)) return rc;
    FunctionT fn = nullptr;
    if (int rc = check(runtime().moduleGetFunction(&fn, module, name_), name_)) return rc;
    functions_[device].store(fn, std::memory_order_release);
    cached = fn;
  }
  *function = cached;
  return 0;
}

int launchRaw(DeviceKernel& kernel, Dim3 grid, Dim3 block, unsigned lds_bytes, void* stream,
              void** args) {
  void* fn = nullptr;
  if (int rc = kernel.resolve(&fn)) return rc;
  return check(runtime().moduleLaunchKernel(fn, grid.x, grid.y, grid.z, block.x, block.y, block.z,
                                            lds_bytes, stream, args, nullptr),
               kernel.name());
}

int launchResidentRaw(DeviceKernel& kernel, Dim3 grid, Dim3 block, unsigned lds_bytes,
                      void* stream, void** args) {
  void* fn = nullptr;
  if (int rc = kernel.resolve(&fn)) return rc;
  int per_cu = 0;
  if (int rc = check(runtime().moduleOccupancy(&per_cu, fn,
                                               static_cast<int>(block.x * block.y * block.z),
                                               lds_bytes),
                     "hipModuleOccupancyMaxActiveBlocksPerMultiprocessor"))
    return rc;
  int cus = 0;
  if (int rc = computeUnits(&cus)) return rc;
  if (static_cast<int64_t>(grid.x) * grid.y * grid.z > static_cast<int64_t>(per_cu) * cus)
    return fail(DLI_HIP_EINVAL, std::string(kernel.name()) + ": " +
                                    std::to_string(grid.x * grid.y * grid.z) +
                                    " workgroups cannot all be resident (" +
                                    std::to_string(per_cu) + " per CU, " + std::to_string(cus) +
                                    " CUs)");
  // A plain launch, eager or captured alike. The grid fits the device at once (checked above),
  // so on a device that runs nothing else every workgroup is resident together; work on other
  // streams can only delay some workgroups, and the kernel's bounded waits turn a wait that
  // outlasts that into a reported give-up, never a hang. (hipModuleLaunchCooperativeKernel
  // was used for eager launches before: under rocprofv3 its runtime path made every profiled
  // process end with a SIGSEGV in the profiler's teardown.)
  return check(runtime().moduleLaunchKernel(fn, grid.x, grid.y, grid.z, block.x, block.y, block.z,
                                            lds_bytes, stream, args, nullptr),
               kernel.name());
}

int moduleGlobal(const char* module, const char* name, void** ptr, size_t* bytes) {
  if (int rc = requireRuntime()) return rc;
  int device = 0;
  if (int rc = check(runtime().getDevice(&device), "hipGetDevice")) return rc;
  ModuleT loaded = nullptr;
  if (int rc = loadEmbeddedModule(device, module, &loaded)) return rc;
  return check(runtime().moduleGetGlobal(ptr, bytes, loaded, name), "hipModuleGetGlobal");
}

}  // namespace dli::hip

using dli::hip::check;
using dli::hip::fail;
using dli::hip::requireRuntime;
using dli::hip::runtime;

extern "C" {

int dli_hip_available(void) { return requireRuntime() == 0 ? 1 : 0; }

const char* dli_hip_load_error(void) { return runtime().load_error.c_str(); }

const char* dli_hip_last_error(void) { return dli::hip::t_last_error.c_str(); }

const char* dli_hip_target_arch(void) { return DLI_HIP_TARGET_ARCH; }

int dli_hip_device_count(int* count) {
  if (count == nullptr) return fail(DLI_HIP_EINVAL, "count is NULL");
  *count = runtime().device_count;
  return requireRuntime();
}

int dli_hip_get_device(int* device) {
  if (device == nullptr) return fail(DLI_HIP_EINVAL, "device is NULL");
  if (int rc = requireRuntime()) return rc;
  return check(runtime().getDevice(device), "hipGetDevice");
}

int dli_hip_compute_units(int* count) {
  if (count == nullptr) return fail(DLI_HIP_EINVAL, "count is NULL");
  return dli::hip::computeUnits(count);
}

int dli_hip_set_device(int device) {
  if (int rc = requireRuntime()) return rc;
  return check(runtime().setDevice(device), "hipSetDevice");
}

int dli_hip_code_object(const char* name, const void** image, size_t* image_bytes) {
  if (name == nullptr || image == nullptr || image_bytes == nullptr)
    return fail(DLI_HIP_EINVAL, "name, image and image_bytes must be non-NULL");
  for (const dli::hip::CodeObject& co : dli::hip::kCodeObjects) {
    if (std::strcmp(co.name, name) != 0) continue;
    *image = co.begin;
    *image_bytes = static_cast<size_t>(co.end - co.begin);
    return 0;
  }
  return fail(DLI_HIP_EINVAL, std::string("no embedded code object named ") + name);
}

int dli_hip_module_load(const void* image, size_t image_bytes, void** module) {
  if (image == nullptr || image_bytes == 0 || module == nullptr)
    return fail(DLI_HIP_EINVAL, "module image is empty");
  if (int rc = requireRuntime()) return rc;
  return check(runtime().moduleLoadData(module, image), "hipModuleLoadData");
}

int dli_hip_module_get_function(void* module, const char* name, void** function) {
  if (module == nullptr || name == nullptr || function == nullptr)
    return fail(DLI_HIP_EINVAL, "module, name and function must be non-NULL");
  if (int rc = requireRuntime()) return rc;
  return check(runtime().moduleGetFunction(function, module, name), "hipModuleGetFunction");
}

int dli_hip_module_unload(void* module) {
  if (module == nullptr) return 0;
  if (int rc = requireRuntime()) return rc;
  return check(runtime().moduleUnload(module), "hipModuleUnload");
}

int dli_hip_launch(void* function, unsigned grid_x, unsigned grid_y, unsigned grid_z,
                   unsigned block_x, unsigned block_y, unsigned block_z, unsigned lds_bytes,
                   void* stream, void** args) {
  if (grid_x == 0 || grid_y == 0 || grid_z == 0) return 0;
  if (function == nullptr) return fail(DLI_HIP_EINVAL, "kernel function is NULL");
  if (int rc = requireRuntime()) return rc;
  return check(runtime().moduleLaunchKernel(function, grid_x, grid_y, grid_z, block_x, block_y,
                                            block_z, lds_bytes, stream, args, nullptr),
               "hipModuleLaunchKernel");
}

int dli_hip_malloc(size_t bytes, void** ptr) {
  if (ptr == nullptr) return fail(DLI_HIP_EINVAL, "ptr is NULL");
  *ptr = nullptr;
  if (int rc = requireRuntime()) return rc;
  return check(runtime().malloc_(ptr, bytes), "hipMalloc");
}

int dli_hip_free(void* ptr) {
  if (ptr == nullptr) return 0;
  if (int rc = requireRuntime()) return rc;
  return check(runtime().free_(ptr), "hipFree");
}

int dli_hip_memcpy(void* dst, const void* src, size_t bytes, int kind) {
  if (bytes == 0) return 0;
  if (int rc = requireRuntime()) return rc;
  return check(runtime().memcpy_(dst, src, bytes, kind), "hipMemcpy");
}

int dli_hip_memcpy_async(void* dst, const void* src, size_t bytes, int kind, void* stream) {
  if (bytes == 0) return 0;
  if (int rc = requireRuntime()) return rc;
  return check(runtime().memcpyAsync(dst, src, bytes, kind, stream), "hipMemcpyAsync");
}

int dli_hip_stream_synchronize(void* stream) {
  if (int rc = requireRuntime()) return rc;
  return check(runtime().streamSynchronize(stream), "hipStreamSynchronize");
}

int dli_hip_device_synchronize(void) {
  if (int rc = requireRuntime()) return rc;
  return check(runtime().deviceSynchronize(), "hipDeviceSynchronize");
}

int dli_hip_event_create(void** event) {
  if (event == nullptr) return fail(DLI_HIP_EINVAL, "event is NULL");
  if (int rc = requireRuntime()) return rc;
  return check(runtime().eventCreate(event), "hipEventCreate");
}

int dli_hip_event_record(void* event, void* stream) {
  if (int rc = requireRuntime()) return rc;
  return check(runtime().eventRecord(event, stream), "hipEventRecord");
}

int dli_hip_event_synchronize(void* event) {
  if (int rc = requireRuntime()) return rc;
  return check(runtime().eventSynchronize(event), "hipEventSynchronize");
}

int dli_hip_event_elapsed_ms(void* start, void* stop, float* ms) {
  if (ms == nullptr) return fail(DLI_HIP_EINVAL, "ms is NULL");
  if (int rc = requireRuntime()) return rc;
  return check(runtime().eventElapsedTime(ms, start, stop), "hipEventElapsedTime");
}

int dli_hip_stream_is_capturing(void* stream, int* capturing) {
  if (capturing == nullptr) return fail(DLI_HIP_EINVAL, "capturing is NULL");
  if (int rc = requireRuntime()) return rc;
  int status = 0;  // hipStreamCaptureStatus: 0 none, 1 active, 2 invalidated
  if (int rc = check(runtime().streamIsCapturing(stream, &status), "hipStreamIsCapturing"))
    return rc;
  *capturing = status != 0 ? 1 : 0;
  return 0;
}

int dli_hip_event_destroy(void* event) {
  if (event == nullptr) return 0;
  if (int rc = requireRuntime()) return rc;
  return check(runtime().eventDestroy(event), "hipEventDestroy");
}

}  // extern "C"
