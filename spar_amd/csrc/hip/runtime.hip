// Device runtime of the gfx950 backend: device selection, one stream per
// device, a caching allocator, copies, zero fill, event timing and error text.
//
// Replaces src/backend/cuda_runtime.cppm:121-345 (cudaMalloc per tensor,
// synchronous cudaMemcpy/cudaMemset) and the launch prologue/epilogue of
// src/backend/cuda_kernels.cu:24-49 (select_device, cudaDeviceSynchronize).
#include <hip/hip_runtime.h>

#include <map>
#include <mutex>
#include <unordered_map>
#include <vector>

#include "common.hpp"

namespace spar_hip {
namespace {

// Small requests are rounded to 512 B, large ones to 2 MiB, so repeated
// tensor shapes map to the same size class and are served from the cache.
constexpr uint64_t kSmallLimit = uint64_t{1} << 20;
constexpr uint64_t kSmallRound = 512;
constexpr uint64_t kLargeRound = uint64_t{2} << 20;

uint64_t rounded_size(uint64_t bytes) {
  const uint64_t round = bytes <= kSmallLimit ? kSmallRound : kLargeRound;
  return (bytes + round - 1) / round * round;
}

struct DeviceState {
  std::mutex mutex;
  hipStream_t stream = nullptr;
  int multiprocessors = 0;
  std::multimap<uint64_t, void*> free_blocks;       // size -> block
  std::unordered_map<void*, uint64_t> live_blocks;  // block -> size
  SparHipMemoryStats stats{};
};

std::mutex g_devices_mutex;
std::vector<DeviceState*> g_devices;
int g_device_count = -1;

hipError_t device_count(int* count) {
  std::lock_guard<std::mutex> lock(g_devices_mutex);
  if (g_device_count < 0) {
    int value = 0;
    const hipError_t error = hipGetDeviceCount(&value);
    if (error != hipSuccess) return error;
    g_device_count = value;
    g_devices.assign(static_cast<size_t>(value), nullptr);
  }
  *count = g_device_count;
  return hipSuccess;
}

// Returns the state for a valid device index, or nullptr.
DeviceState* state_for(int device) {
  int count = 0;
  if (device_count(&count) != hipSuccess || device < 0 || device >= count) return nullptr;
  std::lock_guard<std::mutex> lock(g_devices_mutex);
  DeviceState*& slot = g_devices[static_cast<size_t>(device)];
  if (slot == nullptr) slot = new DeviceState();  // lives until process exit
  return slot;
}

// Releases every cached block of `state` back to the driver.  The caller
// holds state->mutex and has made the device current.
hipError_t release_cached(DeviceState* state) {
  hipError_t first = hipSuccess;
  if (state->stream != nullptr) {
    const hipError_t error = hipStreamSynchronize(state->stream);
    if (error != hipSuccess) first = error;
  }
  for (auto& entry : state->free_blocks) {
    const hipError_t error = hipFree(entry.second);
    if (error != hipSuccess && first == hipSuccess) first = error;
    state->stats.bytes_reserved -= entry.first;
    state->stats.bytes_cached -= entry.first;
  }
  state->free_blocks.clear();
  return first;
}

hipError_t allocate_on(DeviceState* state, void** pointer, uint64_t bytes) {
  const uint64_t size = rounded_size(bytes);
  std::lock_guard<std::mutex> lock(state->mutex);
  // Best fit among cached blocks, but never hand out a block more than twice
  // the request (large tensors would otherwise pin much larger blocks).
  auto found = state->free_blocks.lower_bound(size);
  if (found != state->free_blocks.end() && found->first <= 2 * size) {
    *pointer = found->second;
    state->live_blocks.emplace(found->second, found->first);
    state->stats.bytes_cached -= found->first;
    state->stats.bytes_in_use += found->first;
    state->stats.cache_hits += 1;
    state->free_blocks.erase(found);
    return hipSuccess;
  }
  void* block = nullptr;
  hipError_t error = hipMalloc(&block, size);
  if (error == hipErrorOutOfMemory || error == hipErrorMemoryAllocation) {
    (void)hipGetLastError();
    const hipError_t released = release_cached(state);
    if (released != hipSuccess) {
      (void)hipGetLastError();
      return released;
    }
    error = hipMalloc(&block, size);
  }
  if (error != hipSuccess) {
    (void)hipGetLastError();
    return error;
  }
  *pointer = block;
  state->live_blocks.emplace(block, size);
  state->stats.bytes_in_use += size;
  state->stats.bytes_reserved += size;
  state->stats.device_allocations += 1;
  return hipSuccess;
}

void release_on(DeviceState* state, void* pointer) {
  std::lock_guard<std::mutex> lock(state->mutex);
  auto found = state->live_blocks.find(pointer);
  if (found == state->live_blocks.end()) return;
  const uint64_t size = found->second;
  state->live_blocks.erase(found);
  state->free_blocks.emplace(size, pointer);
  state->stats.bytes_in_use -= size;
  state->stats.bytes_cached += size;
}

// Zero fill: 16-byte stores over the aligned body, bytes for the tail.
__global__ void __launch_bounds__(256) zero_kernel(uint4* body, uint64_t vector_count,
                                                   unsigned char* tail, uint32_t tail_bytes) {
  const uint64_t stride = static_cast<uint64_t>(gridDim.x) * blockDim.x;
  for (uint64_t i = static_cast<uint64_t>(blockIdx.x) * blockDim.x + threadIdx.x;
       i < vector_count; i += stride) {
    body[i] = make_uint4(0, 0, 0, 0);
  }
  if (blockIdx.x == 0 && threadIdx.x < tail_bytes) tail[threadIdx.x] = 0;
}

// Reads every 16-byte word of a buffer with ordinary (cached) loads.  Any
// dirty lines the reads evict are written back during this kernel, so a
// timed kernel launched afterwards starts from a cold, clean cache.
__global__ void __launch_bounds__(256) touch_kernel(const uint4* words, uint64_t count,
                                                    unsigned* sink) {
  unsigned acc = 0;
  const uint64_t stride = static_cast<uint64_t>(gridDim.x) * blockDim.x;
  for (uint64_t i = static_cast<uint64_t>(blockIdx.x) * blockDim.x + threadIdx.x; i < count;
       i += stride) {
    const uint4 w = words[i];
    acc ^= w.x ^ w.y ^ w.z ^ w.w;
  }
  // Written only for an impossible pattern so the loads cannot be elided.
  if (acc == 0x9E3779B9u && sink != nullptr) *sink = acc;
}

__global__ void __launch_bounds__(256) zero_bytes_kernel(unsigned char* bytes, uint64_t count) {
  const uint64_t stride = static_cast<uint64_t>(gridDim.x) * blockDim.x;
  for (uint64_t i = static_cast<uint64_t>(blockIdx.x) * blockDim.x + threadIdx.x; i < count;
       i += stride) {
    bytes[i] = 0;
  }
}

}  // namespace

DeviceGuard::~DeviceGuard() {
  if (changed) (void)hipSetDevice(previous);
}

hipError_t enter(int device, DeviceGuard& guard) {
  static_cast<void>(hipGetLastError());
  DeviceState* state = state_for(device);
  if (state == nullptr) {
    guard.error = hipErrorInvalidDevice;
    return guard.error;
  }
  hipError_t error = hipGetDevice(&guard.previous);
  if (error != hipSuccess) return guard.error = error;
  if (guard.previous != device) {
    error = hipSetDevice(device);
    if (error != hipSuccess) return guard.error = error;
    guard.changed = true;
  }
  {
    std::lock_guard<std::mutex> lock(state->mutex);
    if (state->stream == nullptr) {
      error = hipStreamCreateWithFlags(&state->stream, hipStreamNonBlocking);
      if (error != hipSuccess) return guard.error = error;
      int value = 0;
      if (hipDeviceGetAttribute(&value, hipDeviceAttributeMultiprocessorCount, device) ==
              hipSuccess &&
          value > 0) {
        state->multiprocessors = value;
      } else {
        state->multiprocessors = 256;
      }
    }
    guard.stream = state->stream;
    guard.multiprocessors = state->multiprocessors;
  }
  return hipSuccess;
}

SparHipStatus finish(const DeviceGuard& guard) {
  (void)guard;
  const hipError_t error = hipGetLastError();
  return error == hipSuccess ? ok() : runtime(error);
}

hipError_t scratch_allocate(void** pointer, uint64_t bytes, int device) {
  DeviceState* state = state_for(device);
  if (state == nullptr) return hipErrorInvalidDevice;
  return allocate_on(state, pointer, bytes);
}

void scratch_release(void* pointer, int device) {
  DeviceState* state = state_for(device);
  if (state != nullptr && pointer != nullptr) release_on(state, pointer);
}

}  // namespace spar_hip

using namespace spar_hip;

extern "C" SparHipStatus spar_hip_device_count(int* count) {
  if (count == nullptr) return invalid();
  const hipError_t error = spar_hip::device_count(count);
  return error == hipSuccess ? ok() : runtime(error);
}

extern "C" SparHipStatus spar_hip_multiprocessor_count(int* count, int device) {
  if (count == nullptr) return invalid();
  DeviceGuard guard;
  if (enter(device, guard) != hipSuccess) return runtime(guard.error);
  *count = guard.multiprocessors;
  return ok();
}

extern "C" SparHipStatus spar_hip_allocate(void** pointer, uint64_t bytes, int device) {
  if (pointer == nullptr) return invalid();
  *pointer = nullptr;
  if (bytes == 0) return ok();
  DeviceGuard guard;
  if (enter(device, guard) != hipSuccess) return runtime(guard.error);
  const hipError_t error = scratch_allocate(pointer, bytes, device);
  return error == hipSuccess ? ok() : runtime(error);
}

extern "C" SparHipStatus spar_hip_deallocate(void* pointer, int device) {
  if (pointer == nullptr) return ok();
  DeviceState* state = state_for(device);
  if (state == nullptr) return runtime(hipErrorInvalidDevice);
  release_on(state, pointer);
  return ok();
}

extern "C" SparHipStatus spar_hip_empty_cache(int device) {
  DeviceGuard guard;
  if (enter(device, guard) != hipSuccess) return runtime(guard.error);
  DeviceState* state = state_for(device);
  std::lock_guard<std::mutex> lock(state->mutex);
  const hipError_t error = release_cached(state);
  return error == hipSuccess ? ok() : runtime(error);
}

extern "C" SparHipStatus spar_hip_memory_stats(SparHipMemoryStats* stats, int device) {
  if (stats == nullptr) return invalid();
  DeviceState* state = state_for(device);
  if (state == nullptr) return runtime(hipErrorInvalidDevice);
  std::lock_guard<std::mutex> lock(state->mutex);
  *stats = state->stats;
  return ok();
}

extern "C" SparHipStatus spar_hip_zero(void* destination, uint64_t bytes, int device) {
  if (bytes != 0 && destination == nullptr) return invalid();
  if (bytes == 0) return ok();
  DeviceGuard guard;
  if (enter(device, guard) != hipSuccess) return runtime(guard.error);
  const uint32_t max_blocks = static_cast<uint32_t>(guard.multiprocessors) * 8U;
  if (aligned16(destination)) {
    const uint64_t vectors = bytes / 16;
    const uint32_t tail = static_cast<uint32_t>(bytes % 16);
    uint64_t blocks = (vectors + 255) / 256;
    if (blocks == 0) blocks = 1;
    if (blocks > max_blocks) blocks = max_blocks;
    zero_kernel<<<static_cast<uint32_t>(blocks), 256, 0, guard.stream>>>(
        static_cast<uint4*>(destination), vectors,
        static_cast<unsigned char*>(destination) + vectors * 16, tail);
  } else {
    uint64_t blocks = (bytes + 255) / 256;
    if (blocks > max_blocks) blocks = max_blocks;
    zero_bytes_kernel<<<static_cast<uint32_t>(blocks), 256, 0, guard.stream>>>(
        static_cast<unsigned char*>(destination), bytes);
  }
  return finish(guard);
}

extern "C" SparHipStatus spar_hip_touch(const void* buffer, uint64_t bytes, void* sink,
                                        int device) {
  if (bytes != 0 && (buffer == nullptr || !aligned16(buffer) || bytes % 16 != 0)) return invalid();
  if (bytes == 0) return ok();
  DeviceGuard guard;
  if (enter(device, guard) != hipSuccess) return runtime(guard.error);
  const uint32_t blocks = static_cast<uint32_t>(guard.multiprocessors) * 8U;
  touch_kernel<<<blocks, 256, 0, guard.stream>>>(static_cast<const uint4*>(buffer), bytes / 16,
                                                 static_cast<unsigned*>(sink));
  return finish(guard);
}

extern "C" SparHipStatus spar_hip_copy_host_to_device(void* destination, const void* source,
                                                      uint64_t bytes, int device) {
  if (bytes != 0 && (destination == nullptr || source == nullptr)) return invalid();
  if (bytes == 0) return ok();
  DeviceGuard guard;
  if (enter(device, guard) != hipSuccess) return runtime(guard.error);
  hipError_t error =
      hipMemcpyAsync(destination, source, bytes, hipMemcpyHostToDevice, guard.stream);
  if (error == hipSuccess) error = hipStreamSynchronize(guard.stream);
  return error == hipSuccess ? ok() : runtime(error);
}

extern "C" SparHipStatus spar_hip_copy_device_to_host(void* destination, const void* source,
                                                      uint64_t bytes, int device) {
  if (bytes != 0 && (destination == nullptr || source == nullptr)) return invalid();
  if (bytes == 0) return ok();
  DeviceGuard guard;
  if (enter(device, guard) != hipSuccess) return runtime(guard.error);
  hipError_t error =
      hipMemcpyAsync(destination, source, bytes, hipMemcpyDeviceToHost, guard.stream);
  if (error == hipSuccess) error = hipStreamSynchronize(guard.stream);
  return error == hipSuccess ? ok() : runtime(error);
}

extern "C" SparHipStatus spar_hip_copy_device_to_device(void* destination, int destination_device,
                                                        const void* source, int source_device,
                                                        uint64_t bytes) {
  if (bytes != 0 && (destination == nullptr || source == nullptr)) return invalid();
  if (bytes == 0) return ok();
  if (destination_device == source_device) {
    DeviceGuard guard;
    if (enter(destination_device, guard) != hipSuccess) return runtime(guard.error);
    const hipError_t error =
        hipMemcpyAsync(destination, source, bytes, hipMemcpyDeviceToDevice, guard.stream);
    return error == hipSuccess ? ok() : runtime(error);
  }
  // Cross-device, without a host wait: the peer copy runs on the
  // destination's stream after the source stream's pending work (event
  // `ready`), and the source stream waits for the copy (event `copied`) before
  // anything later on it, such as a kernel that reuses the source block after
  // the caller frees it, can touch the source.
  DeviceGuard source_guard;
  if (enter(source_device, source_guard) != hipSuccess) return runtime(source_guard.error);
  const hipStream_t source_stream = source_guard.stream;
  hipEvent_t ready = nullptr;
  hipError_t error = hipEventCreateWithFlags(&ready, hipEventDisableTiming);
  if (error == hipSuccess) error = hipEventRecord(ready, source_stream);
  if (error != hipSuccess) {
    if (ready != nullptr) static_cast<void>(hipEventDestroy(ready));
    return runtime(error);
  }
  hipEvent_t copied = nullptr;
  {
    DeviceGuard guard;
    if (enter(destination_device, guard) != hipSuccess) {
      static_cast<void>(hipEventDestroy(ready));
      return runtime(guard.error);
    }
    error = hipStreamWaitEvent(guard.stream, ready, 0);
    if (error == hipSuccess) {
      error = hipMemcpyPeerAsync(destination, destination_device, source, source_device, bytes,
                                 guard.stream);
    }
    if (error == hipSuccess) error = hipEventCreateWithFlags(&copied, hipEventDisableTiming);
    if (error == hipSuccess) error = hipEventRecord(copied, guard.stream);
  }
  static_cast<void>(hipEventDestroy(ready));
  if (error == hipSuccess) error = hipStreamWaitEvent(source_stream, copied, 0);
  if (copied != nullptr) static_cast<void>(hipEventDestroy(copied));
  return error == hipSuccess ? ok() : runtime(error);
}

extern "C" SparHipStatus spar_hip_synchronize(int device) {
  DeviceGuard guard;
  if (enter(device, guard) != hipSuccess) return runtime(guard.error);
  const hipError_t error = hipStreamSynchronize(guard.stream);
  return error == hipSuccess ? ok() : runtime(error);
}

extern "C" SparHipStatus spar_hip_stream(void** stream, int device) {
  if (stream == nullptr) return invalid();
  DeviceGuard guard;
  if (enter(device, guard) != hipSuccess) return runtime(guard.error);
  *stream = guard.stream;
  return ok();
}

extern "C" SparHipStatus spar_hip_event_create(void** event) {
  if (event == nullptr) return invalid();
  hipEvent_t created = nullptr;
  const hipError_t error = hipEventCreate(&created);
  *event = created;
  return error == hipSuccess ? ok() : runtime(error);
}

extern "C" SparHipStatus spar_hip_event_destroy(void* event) {
  if (event == nullptr) return ok();
  const hipError_t error = hipEventDestroy(static_cast<hipEvent_t>(event));
  return error == hipSuccess ? ok() : runtime(error);
}

extern "C" SparHipStatus spar_hip_event_record(void* event, int device) {
  if (event == nullptr) return invalid();
  DeviceGuard guard;
  if (enter(device, guard) != hipSuccess) return runtime(guard.error);
  const hipError_t error = hipEventRecord(static_cast<hipEvent_t>(event), guard.stream);
  return error == hipSuccess ? ok() : runtime(error);
}

extern "C" SparHipStatus spar_hip_event_elapsed(float* milliseconds, void* start, void* stop) {
  if (milliseconds == nullptr || start == nullptr || stop == nullptr) return invalid();
  hipError_t error = hipEventSynchronize(static_cast<hipEvent_t>(stop));
  if (error == hipSuccess) {
    error = hipEventElapsedTime(milliseconds, static_cast<hipEvent_t>(start),
                                static_cast<hipEvent_t>(stop));
  }
  return error == hipSuccess ? ok() : runtime(error);
}

extern "C" const char* spar_hip_error_string(int hip_error) {
  return hipGetErrorString(static_cast<hipError_t>(hip_error));
}
