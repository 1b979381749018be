// The restore's host side: copy a table's written slot ranges into one contiguous run of rows,
// on several host threads (the reference does it with torch.index_select,
// core/everserve/state/mirror.py:926-932). The source is a store table, [num_slots, row_bytes],
// in memory or mapped from its file; the destination is pinned memory the next H2D copy reads.
// Measured and rejected: reading the file with pread on the same threads. It costs no page
// faults and no mapping to tear down, but the kernel's copy writes through the cache, and with
// the DMA engine reading the other buffer the restore ran at 38 GB/s against 41-55 GB/s here.

#include <algorithm>
#include <cstring>
#include <thread>
#include <vector>

#include "common.hpp"

// 1: the rows are written with nontemporal stores. A plain store first reads every line it
// writes into the cache (a third stream of host memory traffic beside the table's reads and the
// DMA engine's), and leaves the pinned lines dirty in the copying core's cache.
#ifndef EVS_HOST_NT_STORES
#define EVS_HOST_NT_STORES 1
#endif

namespace evs {
namespace {

constexpr int64_t kMinBytesPerThread = int64_t{4} << 20;  // below this a thread costs more than it copies

typedef long long v2i64 __attribute__((ext_vector_type(2)));

// memcpy with 16-byte nontemporal stores where dst is 16-byte aligned; plain copies for the
// unaligned head and the tail.
void stream_copy(char* dst, const char* src, size_t bytes) {
  size_t head = (16 - (reinterpret_cast<uintptr_t>(dst) & 15)) & 15;
  if (head > bytes) head = bytes;
  std::memcpy(dst, src, head);
  size_t i = head;
  for (; i + 64 <= bytes; i += 64) {
    v2i64 w[4];
    std::memcpy(w, src + i, 64);
    for (int k = 0; k < 4; k++)
      __builtin_nontemporal_store(w[k], reinterpret_cast<v2i64*>(dst + i) + k);
  }
  for (; i + 16 <= bytes; i += 16) {
    v2i64 w;
    std::memcpy(&w, src + i, 16);
    __builtin_nontemporal_store(w, reinterpret_cast<v2i64*>(dst + i));
  }
  std::memcpy(dst + i, src + i, bytes - i);
}

void copy_bytes(char* dst, const char* src, size_t bytes) {
  if (EVS_HOST_NT_STORES)
    stream_copy(dst, src, bytes);
  else
    std::memcpy(dst, src, bytes);
}

// Copy output rows [r0, r1) of the concatenated ranges.
void copy_rows(const char* src, int64_t row_bytes, const int64_t* starts, const int64_t* counts,
               const int64_t* first_row, int64_t nranges, char* dst, int64_t r0, int64_t r1) {
  // the range that holds output row r0
  int64_t lo = 0, hi = nranges - 1;
  while (lo < hi) {
    const int64_t mid = (lo + hi + 1) / 2;
    if (first_row[mid] <= r0) lo = mid; else hi = mid - 1;
  }
  int64_t r = r0;
  for (int64_t k = lo; k < nranges && r < r1; k++) {
    const int64_t in_range = r - first_row[k];
    const int64_t take = std::min(counts[k] - in_range, r1 - r);
    if (take <= 0) continue;
    copy_bytes(dst + r * row_bytes, src + (starts[k] + in_range) * row_bytes,
               static_cast<size_t>(take * row_bytes));
    r += take;
  }
  // nontemporal stores are weakly ordered: drain them before the caller learns the copy is done
  if (EVS_HOST_NT_STORES) __builtin_ia32_sfence();
}

// Checks every range against the table's rows and dst's room, and fills first_row (the output
// row each range starts at); the row total is first_row[nranges].
int check_ranges(const char* name, int64_t table_rows, const int64_t* starts,
                 const int64_t* counts, int64_t nranges, int64_t dst_rows,
                 std::vector<int64_t>* first_row) {
  first_row->assign(static_cast<size_t>(nranges) + 1, 0);
  for (int64_t k = 0; k < nranges; k++) {
    EVS_REQUIRE(starts[k] >= 0 && counts[k] >= 0, "%s: negative range %lld", name,
                static_cast<long long>(k));
    EVS_REQUIRE(starts[k] <= table_rows && counts[k] <= table_rows - starts[k],
                "%s: range %lld (%lld + %lld) lies outside the table's %lld rows", name,
                static_cast<long long>(k), static_cast<long long>(starts[k]),
                static_cast<long long>(counts[k]), static_cast<long long>(table_rows));
    EVS_REQUIRE(counts[k] <= dst_rows - (*first_row)[k],
                "%s: the ranges hold more rows than dst's %lld", name,
                static_cast<long long>(dst_rows));
    (*first_row)[k + 1] = (*first_row)[k] + counts[k];
  }
  return EVS_OK;
}

int64_t threads_for(int64_t bytes, int64_t max_threads) {
  const int64_t t = bytes / kMinBytesPerThread;
  return t < 1 ? 1 : (t > max_threads ? max_threads : t);
}

}  // namespace
}  // namespace evs

extern "C" int evs_host_gather_ranges(const void* src, int64_t src_rows, int64_t row_bytes,
                                      const int64_t* starts, const int64_t* counts,
                                      int64_t nranges, void* dst, int64_t dst_rows,
                                      int64_t max_threads, int64_t* rows_out) {
  evs::clear_error();
  if (rows_out != nullptr) *rows_out = 0;
  EVS_REQUIRE(row_bytes > 0 && nranges >= 0 && max_threads >= 1 && src_rows >= 0 &&
                  dst_rows >= 0,
              "evs_host_gather_ranges: row_bytes > 0, nranges >= 0, max_threads >= 1 and "
              "src_rows, dst_rows >= 0");
  EVS_REQUIRE(nranges == 0 || (src != nullptr && dst != nullptr && starts != nullptr &&
                               counts != nullptr),
              "evs_host_gather_ranges: null pointer");
  // every range is checked before anything is copied
  std::vector<int64_t> first_row;
  const int rc = evs::check_ranges("evs_host_gather_ranges", src_rows, starts, counts, nranges,
                                   dst_rows, &first_row);
  if (rc != EVS_OK) return rc;
  const int64_t rows = first_row[nranges];
  if (rows_out != nullptr) *rows_out = rows;  // the copy below cannot fail
  if (rows == 0) return EVS_OK;
  const int64_t threads = evs::threads_for(rows * row_bytes, max_threads);
  const char* s = static_cast<const char*>(src);
  char* d = static_cast<char*>(dst);
  if (threads == 1) {
    evs::copy_rows(s, row_bytes, starts, counts, first_row.data(), nranges, d, 0, rows);
    return EVS_OK;
  }
  std::vector<std::thread> pool;
  pool.reserve(static_cast<size_t>(threads));
  for (int64_t t = 0; t < threads; t++) {
    const int64_t r0 = rows * t / threads;
    const int64_t r1 = rows * (t + 1) / threads;
    pool.emplace_back(evs::copy_rows, s, row_bytes, starts, counts, first_row.data(), nranges, d,
                      r0, r1);
  }
  for (auto& th : pool) th.join();
  return EVS_OK;
}
