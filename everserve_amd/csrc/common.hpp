// Shared pieces of libeverserve_mi355x: the per-thread error message, HIP error checks and an
// exact 32-bit divider for index arithmetic inside kernels.
#pragma once

#include <hip/hip_runtime.h>

#include <cstdint>
#include <cstdio>
#include <string>

#include "everserve_mi355x.h"

namespace evs {

// The message evs_last_error() returns; one per calling thread.
void set_error(const char* fmt, ...) __attribute__((format(printf, 1, 2)));
void clear_error();

#define EVS_REQUIRE(cond, ...)        \
  do {                                \
    if (!(cond)) {                    \
      ::evs::set_error(__VA_ARGS__);  \
      return EVS_EINVAL;              \
    }                                 \
  } while (0)

// A failed call's error is reported here, and read out of HIP's per-thread last error, so that a
// later launch check (EVS_LAUNCHED) does not report it again as its own.
#define EVS_HIP(call)                                                                     \
  do {                                                                                    \
    hipError_t evs_rc_ = (call);                                                          \
    if (evs_rc_ != hipSuccess) {                                                          \
      (void)hipGetLastError();                                                            \
      ::evs::set_error("%s failed: %s (%d)", #call, hipGetErrorString(evs_rc_),          \
                       static_cast<int>(evs_rc_));                                        \
      return EVS_EHIP;                                                                    \
    }                                                                                     \
  } while (0)

// The launch's own error (bad configuration, missing code object) right after enqueueing it.
#define EVS_LAUNCHED(what)                                                                \
  do {                                                                                    \
    hipError_t evs_rc_ = hipGetLastError();                                               \
    if (evs_rc_ != hipSuccess) {                                                          \
      ::evs::set_error("%s launch failed: %s (%d)", what, hipGetErrorString(evs_rc_),    \
                       static_cast<int>(evs_rc_));                                        \
      return EVS_EHIP;                                                                    \
    }                                                                                     \
  } while (0)

inline hipStream_t as_stream(void* s) { return reinterpret_cast<hipStream_t>(s); }

// q = n / d and r = n % d for 0 <= n < 2^31 and 1 <= d < 2^31 with one multiply-high: the
// round-up method (Granlund and Montgomery, "Division by invariant integers using
// multiplication", 1994). m = floor(2^(32+s) / d) + 1 with s = ceil(log2 d) makes
// floor(n * m / 2^(32+s)) == floor(n / d) for every n < 2^31.
struct FastDiv {
  uint32_t d;
  uint32_t m;
  uint32_t s;

  __host__ __device__ FastDiv() : d(1), m(0), s(0) {}
  explicit FastDiv(uint32_t divisor) : d(divisor) {
    s = 0;
    while ((uint64_t{1} << s) < d) ++s;
    m = static_cast<uint32_t>(((uint64_t{1} << (32 + s)) + d - 1) / d - (uint64_t{1} << 32));
    // d a power of two: m == 0 and the quotient is a plain shift
  }
  __host__ __device__ __forceinline__ uint32_t div(uint32_t n) const {
    const uint32_t hi = static_cast<uint32_t>((static_cast<uint64_t>(n) * m) >> 32);
    return (hi + n) >> s;
  }
  __host__ __device__ __forceinline__ void divmod(uint32_t n, uint32_t& q, uint32_t& r) const {
    q = div(n);
    r = n - q * d;
  }
};

inline bool aligned16(int64_t v) { return (v & 15) == 0; }

// Copy `runs` runs of `len` bytes, `spitch` apart in src and `dpitch` apart in dst, on `stream`
// (host code). Runs that lie back to back on both sides go as one hipMemcpyAsync. Pitched runs go
// as one hipMemcpy2DAsync, except device-to-host runs of 1 MiB or more, which go as one
// hipMemcpyAsync each: while the driver clears released device memory in the background (it
// does so on a copy engine, for about a second after 48 GiB was released), a pitched
// device-to-host hipMemcpy2DAsync ran at 15 GB/s on MI355X where hipMemcpyAsync of the same
// bytes ran at 35-56 GB/s; host-to-device pitched copies kept 56 GB/s, and splitting them into
// one copy a run cost a restore 5-20 % in submission gaps.
constexpr int64_t kMinRunCopyBytes = int64_t{1} << 20;
// Which engine moves a copy depends on whether a profiler is attached. Under rocprofv3's kernel
// trace, hipMemcpyAsync between HBM and pinned host memory (32 KiB to 32 MiB, either way) shows
// as a blit kernel on a compute queue and hipMemcpy2DAsync as a DMA-engine copy; without the
// profiler the contiguous device-to-host copy of 640 MiB ran at 56.9 GB/s, the DMA engines'
// rate, against 54.6 GB/s under the trace and with the DMA engines turned off (blit kernels).
// Sending every host copy through hipMemcpy2DAsync was measured against the forms below on a
// Llama-3-8B decode step that stages 8 MiB a step, without the profiler: the snapshot added
// 40-47 us a step either way (10 interleaved rounds of 100 steps).

inline int copy_runs(void* dst, int64_t dpitch, const void* src, int64_t spitch, int64_t len,
                     int64_t runs, hipMemcpyKind kind, hipStream_t stream) {
  if (runs <= 0 || len <= 0) return EVS_OK;
  char* d = static_cast<char*>(dst);
  const char* s = static_cast<const char*>(src);
  if (runs == 1 || (dpitch == len && spitch == len)) {
    EVS_HIP(hipMemcpyAsync(d, s, static_cast<size_t>(len * runs), kind, stream));
  } else if (kind == hipMemcpyDeviceToHost && len >= kMinRunCopyBytes) {
    for (int64_t r = 0; r < runs; r++)
      EVS_HIP(hipMemcpyAsync(d + r * dpitch, s + r * spitch, static_cast<size_t>(len), kind,
                             stream));
  } else {
    EVS_HIP(hipMemcpy2DAsync(d, static_cast<size_t>(dpitch), s, static_cast<size_t>(spitch),
                             static_cast<size_t>(len), static_cast<size_t>(runs), kind, stream));
  }
  return EVS_OK;
}

}  // namespace evs
