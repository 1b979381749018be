// The library's host-side helpers: errors, the region layout constants, pinned and device
// memory, a zero-fill kernel, inter-process handles and the wall-clock rate
// (core/csrc/gather.cu:137-148 and core/csrc/slot.cu:229-232,283-312 in the reference).

#include <cstdarg>
#include <cstring>

#include "common.hpp"

namespace evs {

namespace {
thread_local char g_error[512];
}

void set_error(const char* fmt, ...) {
  va_list ap;
  va_start(ap, fmt);
  vsnprintf(g_error, sizeof(g_error), fmt, ap);
  va_end(ap);
}

void clear_error() { g_error[0] = '\0'; }

int wall_clock_khz(int64_t* khz);  // reduce.hip

namespace {

constexpr int kFillThreads = 256;

// Zero `bytes` bytes: 16-byte words over the aligned middle, single bytes at both ends.
__global__ __launch_bounds__(kFillThreads) void fill_zero(char* p, int64_t bytes) {
  typedef uint32_t u32x4 __attribute__((ext_vector_type(4)));
  const int64_t misalign = (16 - (reinterpret_cast<int64_t>(p) & 15)) & 15;
  const int64_t head = misalign < bytes ? misalign : bytes;
  const int64_t words = (bytes - head) / 16;
  const int64_t tid = static_cast<int64_t>(blockIdx.x) * kFillThreads + threadIdx.x;
  const int64_t stride = static_cast<int64_t>(gridDim.x) * kFillThreads;
  u32x4* w = reinterpret_cast<u32x4*>(p + head);
  for (int64_t i = tid; i < words; i += stride) w[i] = u32x4{0u, 0u, 0u, 0u};
  const int64_t tail_start = head + words * 16;
  if (tid < head) p[tid] = 0;
  if (tid < bytes - tail_start) p[tail_start + tid] = 0;
}

}  // namespace
}  // namespace evs

extern "C" const char* evs_last_error(void) { return evs::g_error; }

extern "C" int evs_layout_constants(int64_t* out, int64_t n) {
  evs::clear_error();
  EVS_REQUIRE(out != nullptr && n >= 5, "evs_layout_constants: needs room for 5 words");
  out[0] = EVS_MAX_ROWS;
  out[1] = EVS_CTRL_WORDS;
  out[2] = EVS_ABORT;
  out[3] = EVS_LATE;
  out[4] = EVS_BOUND;
  return EVS_OK;
}

extern "C" int evs_slot_blocks(int64_t maxn, int64_t words, int64_t* out) {
  evs::clear_error();
  EVS_REQUIRE(out != nullptr, "evs_slot_blocks: null output");
  EVS_REQUIRE(maxn >= 0 && words >= 1, "evs_slot_blocks: maxn >= 0 and words >= 1");
  const int64_t per_block = int64_t{256} * words;
  *out = (maxn / 2 + per_block - 1) / per_block;
  return EVS_OK;
}

extern "C" int evs_host_register_mapped(void* ptr, int64_t bytes, void** device_ptr) {
  evs::clear_error();
  EVS_REQUIRE(ptr != nullptr && bytes > 0 && device_ptr != nullptr,
              "evs_host_register_mapped: null pointer or empty range");
  EVS_HIP(hipHostRegister(ptr, static_cast<size_t>(bytes),
                          hipHostRegisterMapped | hipHostRegisterPortable));
  void* dev = nullptr;
  hipError_t rc = hipHostGetDevicePointer(&dev, ptr, 0);
  if (rc != hipSuccess) {
    (void)hipGetLastError();
    (void)hipHostUnregister(ptr);
    evs::set_error("hipHostGetDevicePointer failed: %s (%d)", hipGetErrorString(rc),
                   static_cast<int>(rc));
    return EVS_EHIP;
  }
  *device_ptr = dev;
  return EVS_OK;
}

extern "C" int evs_host_unregister(void* ptr) {
  evs::clear_error();
  EVS_HIP(hipHostUnregister(ptr));
  return EVS_OK;
}

extern "C" int evs_host_alloc_mapped(int64_t bytes, void** host_ptr, void** device_ptr) {
  evs::clear_error();
  EVS_REQUIRE(bytes > 0 && host_ptr != nullptr && device_ptr != nullptr,
              "evs_host_alloc_mapped: empty or null");
  void* h = nullptr;
  EVS_HIP(hipHostMalloc(&h, static_cast<size_t>(bytes),
                        hipHostMallocMapped | hipHostMallocPortable | hipHostMallocCoherent));
  std::memset(h, 0, static_cast<size_t>(bytes));
  void* dev = nullptr;
  hipError_t rc = hipHostGetDevicePointer(&dev, h, 0);
  if (rc != hipSuccess) {
    (void)hipGetLastError();
    (void)hipHostFree(h);
    evs::set_error("hipHostGetDevicePointer failed: %s (%d)", hipGetErrorString(rc),
                   static_cast<int>(rc));
    return EVS_EHIP;
  }
  *host_ptr = h;
  *device_ptr = dev;
  return EVS_OK;
}

extern "C" int evs_host_free(void* host_ptr) {
  evs::clear_error();
  EVS_HIP(hipHostFree(host_ptr));
  return EVS_OK;
}

extern "C" int evs_device_alloc(int64_t bytes, void** ptr) {
  evs::clear_error();
  EVS_REQUIRE(bytes > 0 && ptr != nullptr, "evs_device_alloc: empty or null");
  void* p = nullptr;
  EVS_HIP(hipMalloc(&p, static_cast<size_t>(bytes)));
  hipError_t rc = hipMemset(p, 0, static_cast<size_t>(bytes));
  if (rc != hipSuccess) {
    (void)hipGetLastError();
    (void)hipFree(p);
    evs::set_error("hipMemset failed: %s (%d)", hipGetErrorString(rc), static_cast<int>(rc));
    return EVS_EHIP;
  }
  *ptr = p;
  return EVS_OK;
}

extern "C" int evs_device_free(void* ptr) {
  evs::clear_error();
  EVS_HIP(hipFree(ptr));
  return EVS_OK;
}

extern "C" int evs_memset_async(void* ptr, int64_t bytes, void* stream) {
  evs::clear_error();
  EVS_REQUIRE(bytes >= 0, "evs_memset_async: negative size");
  if (bytes == 0) return EVS_OK;
  EVS_REQUIRE(ptr != nullptr, "evs_memset_async: null pointer");
  int64_t blocks = (bytes / 16 + evs::kFillThreads - 1) / evs::kFillThreads;
  if (blocks < 1) blocks = 1;
  if (blocks > 4096) blocks = 4096;
  hipLaunchKernelGGL(evs::fill_zero, dim3(static_cast<uint32_t>(blocks)),
                     dim3(evs::kFillThreads), 0, evs::as_stream(stream),
                     static_cast<char*>(ptr), bytes);
  EVS_LAUNCHED("evs_memset_async");
  return EVS_OK;
}

extern "C" int evs_copy_rows_async(void* dst, const void* src, int64_t groups, int64_t bytes,
                                   int64_t pitch, void* stream) {
  evs::clear_error();
  EVS_REQUIRE(groups >= 0 && bytes >= 0 && pitch >= bytes,
              "evs_copy_rows_async: needs groups >= 0 and pitch >= bytes >= 0");
  if (groups == 0 || bytes == 0) return EVS_OK;
  EVS_REQUIRE(dst != nullptr && src != nullptr, "evs_copy_rows_async: null pointer");
  return evs::copy_runs(dst, pitch, src, pitch, bytes, groups, hipMemcpyDefault,
                        evs::as_stream(stream));
}

extern "C" int evs_event_create(int system_fence, void** event) {
  evs::clear_error();
  EVS_REQUIRE(event != nullptr, "evs_event_create: null output");
  hipEvent_t e = nullptr;
  const unsigned flags =
      hipEventDisableTiming | (system_fence ? 0u : static_cast<unsigned>(hipEventDisableSystemFence));
  EVS_HIP(hipEventCreateWithFlags(&e, flags));
  *event = e;
  return EVS_OK;
}

extern "C" int evs_event_destroy(void* event) {
  evs::clear_error();
  EVS_HIP(hipEventDestroy(static_cast<hipEvent_t>(event)));
  return EVS_OK;
}

extern "C" int evs_event_record(void* event, void* stream) {
  evs::clear_error();
  EVS_HIP(hipEventRecord(static_cast<hipEvent_t>(event), evs::as_stream(stream)));
  return EVS_OK;
}

extern "C" int evs_event_synchronize(void* event) {
  evs::clear_error();
  EVS_HIP(hipEventSynchronize(static_cast<hipEvent_t>(event)));
  return EVS_OK;
}

extern "C" int evs_stream_handoff(void* producing, void* waiting, void* event) {
  evs::clear_error();
  EVS_REQUIRE(event != nullptr, "evs_stream_handoff: null event");
  EVS_HIP(hipEventRecord(static_cast<hipEvent_t>(event), evs::as_stream(producing)));
  EVS_HIP(hipStreamWaitEvent(evs::as_stream(waiting), static_cast<hipEvent_t>(event), 0));
  return EVS_OK;
}

extern "C" int evs_ipc_handle(void* ptr, uint8_t* handle_out, int64_t handle_bytes) {
  evs::clear_error();
  EVS_REQUIRE(handle_out != nullptr && handle_bytes == sizeof(hipIpcMemHandle_t),
              "evs_ipc_handle: the handle is %zu bytes", sizeof(hipIpcMemHandle_t));
  hipIpcMemHandle_t h;
  EVS_HIP(hipIpcGetMemHandle(&h, ptr));
  std::memcpy(handle_out, &h, sizeof(h));
  return EVS_OK;
}

extern "C" int evs_ipc_open(const uint8_t* handle, int64_t handle_bytes, void** ptr) {
  evs::clear_error();
  EVS_REQUIRE(handle != nullptr && ptr != nullptr && handle_bytes == sizeof(hipIpcMemHandle_t),
              "evs_ipc_open: not an IPC handle");
  hipIpcMemHandle_t h;
  std::memcpy(&h, handle, sizeof(h));
  void* p = nullptr;
  EVS_HIP(hipIpcOpenMemHandle(&p, h, hipIpcMemLazyEnablePeerAccess));
  *ptr = p;
  return EVS_OK;
}

extern "C" int evs_ipc_close(void* ptr) {
  evs::clear_error();
  EVS_HIP(hipIpcCloseMemHandle(ptr));
  return EVS_OK;
}

extern "C" int evs_wall_clock_khz(int64_t* khz) {
  evs::clear_error();
  EVS_REQUIRE(khz != nullptr, "evs_wall_clock_khz: null output");
  return evs::wall_clock_khz(khz);
}
