// A restore's (slot, staged row) pairs in slot order, on the device: the ordering that lets the
// pair scatter (evs_scatter_pairs in rows.hip) write each layer's cache front to back, for a
// caller whose slot list is already in HBM. The pairs are sorted with rocPRIM's radix sort on
// the low key_bits bits of the slot ids (the cache's slot count fixes how many matter: 18 for
// 262,144 slots). The sort is stable, so equal slots keep their listed order. Everything it needs
// beyond its inputs and outputs lives in a workspace the caller allocates: the row numbers
// 0..n-1, then rocPRIM's temporary storage. rocPRIM clears its counters there with
// hipMemsetAsync, so this call is not one to capture in a HIP graph.
//
// evs_order_pairs_static is the same call for callers that cannot allocate (no workspace
// argument): its scratch is a file-scope device array of a fixed size.

#include <mutex>

#include <rocprim/device/device_radix_sort.hpp>

#include "common.hpp"

namespace evs {
namespace {

constexpr int kIotaThreads = 256;
constexpr int64_t kAlign = 256;

__global__ __launch_bounds__(kIotaThreads) void iota(int64_t* rows, int64_t n) {
  const int64_t i = static_cast<int64_t>(blockIdx.x) * kIotaThreads + threadIdx.x;
  if (i < n) rows[i] = i;
}

int64_t round_up(int64_t v) { return (v + kAlign - 1) / kAlign * kAlign; }

// rocPRIM's temporary storage for n pairs of 64-bit keys and values over `bits` key bits.
int sort_storage(int64_t n, int bits, size_t* bytes) {
  *bytes = 0;
  EVS_HIP(rocprim::radix_sort_pairs(nullptr, *bytes, static_cast<const uint64_t*>(nullptr),
                                    static_cast<uint64_t*>(nullptr),
                                    static_cast<const int64_t*>(nullptr),
                                    static_cast<int64_t*>(nullptr), static_cast<uint32_t>(n), 0u,
                                    static_cast<unsigned>(bits), hipStream_t{nullptr}));
  return EVS_OK;
}

// The allocation-free variant's scratch: the row numbers and rocPRIM's temporary storage of a
// call of up to EVS_ORDER_STATIC_MAX_PAIRS pairs, in a file-scope device array. Every GPU the
// library runs on holds its own copy until the process ends. Host code never passes the array's
// name to a kernel (in host code it is a stand-in, not a device address): the address comes from
// hipGetSymbolAddress, once per device, with that device current.
static __device__ __align__(256) unsigned char scratch[EVS_ORDER_STATIC_SCRATCH_BYTES];

constexpr int kMaxDevices = 64;
std::mutex g_scratch_lock;
void* g_scratch[kMaxDevices];  // the array's address on each device, once looked up

// The current device's copy of the scratch array.
int scratch_here(void** out) {
  int dev = -1;
  EVS_HIP(hipGetDevice(&dev));
  EVS_REQUIRE(dev >= 0 && dev < kMaxDevices, "evs_order_pairs_static: device %d past the %d "
              "devices it keeps a scratch address for", dev, kMaxDevices);
  std::lock_guard<std::mutex> hold(g_scratch_lock);
  if (g_scratch[dev] == nullptr) {
    void* p = nullptr;
    EVS_HIP(hipGetSymbolAddress(&p, HIP_SYMBOL(scratch)));
    EVS_REQUIRE(p != nullptr, "evs_order_pairs_static: no device address for the scratch");
    g_scratch[dev] = p;
  }
  *out = g_scratch[dev];
  return EVS_OK;
}

}  // namespace
}  // namespace evs

extern "C" int evs_order_pairs_workspace(int64_t num_pairs, int key_bits, int64_t* bytes) {
  evs::clear_error();
  EVS_REQUIRE(bytes != nullptr, "evs_order_pairs_workspace: null output");
  EVS_REQUIRE(num_pairs >= 0 && num_pairs < (int64_t{1} << 31),
              "evs_order_pairs_workspace: 0 <= num_pairs < 2^31, got %lld",
              static_cast<long long>(num_pairs));
  EVS_REQUIRE(key_bits >= 1 && key_bits <= 64, "evs_order_pairs_workspace: key_bits in 1..64");
  size_t sort_bytes = 0;
  const int rc = evs::sort_storage(num_pairs, key_bits, &sort_bytes);
  if (rc != EVS_OK) return rc;
  *bytes = evs::round_up(num_pairs * 8) + evs::round_up(static_cast<int64_t>(sort_bytes));
  return EVS_OK;
}

extern "C" int evs_order_pairs(const int64_t* slots, int64_t num_pairs, int key_bits,
                               int64_t* slots_out, int64_t* rows_out, void* workspace,
                               int64_t workspace_bytes, void* stream) {
  evs::clear_error();
  int64_t need = 0;
  const int rc = evs_order_pairs_workspace(num_pairs, key_bits, &need);
  if (rc != EVS_OK) return rc;
  if (num_pairs == 0) return EVS_OK;
  EVS_REQUIRE(slots != nullptr && slots_out != nullptr && rows_out != nullptr &&
                  workspace != nullptr,
              "evs_order_pairs: null pointer");
  EVS_REQUIRE(workspace_bytes >= need,
              "evs_order_pairs: the workspace holds %lld bytes, %lld needed",
              static_cast<long long>(workspace_bytes), static_cast<long long>(need));
  EVS_REQUIRE((reinterpret_cast<uintptr_t>(workspace) & (evs::kAlign - 1)) == 0,
              "evs_order_pairs: the workspace must be %lld-byte aligned",
              static_cast<long long>(evs::kAlign));
  hipStream_t s = evs::as_stream(stream);
  int64_t* rows = static_cast<int64_t*>(workspace);
  char* sort_tmp = static_cast<char*>(workspace) + evs::round_up(num_pairs * 8);
  size_t sort_bytes = static_cast<size_t>(need - evs::round_up(num_pairs * 8));
  const int64_t grid = (num_pairs + evs::kIotaThreads - 1) / evs::kIotaThreads;
  hipLaunchKernelGGL(evs::iota, dim3(static_cast<uint32_t>(grid)), dim3(evs::kIotaThreads), 0, s,
                     rows, num_pairs);
  EVS_LAUNCHED("evs_order_pairs");
  // the slot ids are compared as unsigned on their low key_bits bits: a padding id (negative)
  // lands wherever those bits put it, and the pair scatter skips it
  EVS_HIP(rocprim::radix_sort_pairs(sort_tmp, sort_bytes,
                                    reinterpret_cast<const uint64_t*>(slots),
                                    reinterpret_cast<uint64_t*>(slots_out),
                                    static_cast<const int64_t*>(rows), rows_out,
                                    static_cast<uint32_t>(num_pairs), 0u,
                                    static_cast<unsigned>(key_bits), s));
  return EVS_OK;
}

extern "C" int evs_order_pairs_static(const int64_t* slots, int64_t num_pairs, int key_bits,
                                      int64_t* slots_out, int64_t* rows_out, void* stream) {
  evs::clear_error();
  EVS_REQUIRE(num_pairs >= 0 && num_pairs <= EVS_ORDER_STATIC_MAX_PAIRS,
              "evs_order_pairs_static: %lld pairs, at most %d fit its scratch; give "
              "evs_order_pairs a workspace for more",
              static_cast<long long>(num_pairs), EVS_ORDER_STATIC_MAX_PAIRS);
  int64_t need = 0;
  int rc = evs_order_pairs_workspace(num_pairs, key_bits, &need);
  if (rc != EVS_OK) return rc;
  EVS_REQUIRE(need <= EVS_ORDER_STATIC_SCRATCH_BYTES,
              "evs_order_pairs_static: %lld pairs of %d key bits need %lld bytes of scratch, "
              "it holds %d", static_cast<long long>(num_pairs), key_bits,
              static_cast<long long>(need), EVS_ORDER_STATIC_SCRATCH_BYTES);
  if (num_pairs == 0) return EVS_OK;
  void* ptr = nullptr;  // this device's copy of the scratch array
  rc = evs::scratch_here(&ptr);
  if (rc != EVS_OK) return rc;
  // the row numbers are written whole by the call and rocPRIM clears its own counters, so
  // nothing from the previous call's contents is read
  return evs_order_pairs(slots, num_pairs, key_bits, slots_out, rows_out, ptr,
                         EVS_ORDER_STATIC_SCRATCH_BYTES, stream);
}
