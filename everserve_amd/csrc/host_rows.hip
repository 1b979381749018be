// Host-memory copies of the path, on several host threads with nontemporal stores.
//
// The restore's host side: copy store tables' written slot ranges into contiguous runs of rows
// (the reference does it per table with torch.index_select, core/everserve/state/mirror.py:
// 926-932). A source is a store table, [num_slots, row_bytes], in memory or mapped from its file;
// the destination is pinned memory the next H2D copy reads. Several tables with the same ranges
// (the heads of one layer) are gathered in one call, each into its own block of the destination.
//
// The step's delivery: staged rows in HBM to host memory that cannot be registered with the
// device (a staging file in shared memory, which the node's store maps by name; mirror.py:
// 588-634). The copy engine moves a batch of rows into one of two pinned bounce buffers while
// host threads copy the previous batch out of the other into the destination.
//
// Measured and rejected: reading the file with pread on the same threads. It costs no page
// faults and no mapping to tear down, but the kernel's copy writes through the cache, and with
// the DMA engine reading the other buffer the restore ran at 38 GB/s against 41-55 GB/s here.

#include <algorithm>
#include <cstring>
#include <vector>

#include "common.hpp"
#include "host_copy.hpp"
#include "workers.hpp"

// 1: the rows are written with nontemporal stores. A plain store first reads every line it
// writes into the cache (a third stream of host memory traffic beside the table's reads and the
// DMA engine's), and leaves the pinned lines dirty in the copying core's cache.
#ifndef EVS_HOST_NT_STORES
#define EVS_HOST_NT_STORES 1
#endif

namespace evs {
namespace {

// A gather of fewer bytes than this a thread runs on fewer threads. Table pages mapped afresh
// fault in as they are read (about 30 GB/s on 16 threads, where warm pages copy at 100 and more),
// so a thread is worth waking for 1 MiB: with 4 MiB a thread, the restore's 16 MiB pieces ran on
// 4 threads and a catch-up of 256 tables took 15 ms instead of 7.
constexpr int64_t kMinBytesPerThread = int64_t{1} << 20;

void copy_bytes(char* dst, const char* src, size_t bytes) {
  if (EVS_HOST_NT_STORES)
    stream_copy(dst, src, bytes);
  else
    std::memcpy(dst, src, bytes);
}

// Copy output rows [r0, r1) of the concatenated ranges of one table.
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
}

// One thread's share of a multi-table gather: flat output rows [f0, f1) of tables x rows, table j
// landing at dst + j * dst_rows * row_bytes.
void copy_tables(const char* const* srcs, int64_t rows, int64_t row_bytes, const int64_t* starts,
                 const int64_t* counts, const int64_t* first_row, int64_t nranges, char* dst,
                 int64_t dst_rows, int64_t f0, int64_t f1) {
  while (f0 < f1) {
    const int64_t j = f0 / rows, r0 = f0 % rows;
    const int64_t r1 = std::min(rows, r0 + (f1 - f0));
    copy_rows(srcs[j], row_bytes, starts, counts, first_row, nranges,
              dst + j * dst_rows * row_bytes, r0, r1);
    f0 += r1 - r0;
  }
  // nontemporal stores are weakly ordered: drain them before the caller learns the copy is done
  if (EVS_HOST_NT_STORES) stream_fence();
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

int64_t threads_for(int64_t bytes, int64_t max_threads, int64_t min_bytes = kMinBytesPerThread) {
  const int64_t t = bytes / min_bytes;
  return t < 1 ? 1 : (t > max_threads ? max_threads : t);
}

int gather_tables(const char* name, const void* const* srcs, int64_t num_tables,
                  int64_t src_rows, int64_t row_bytes, const int64_t* starts,
                  const int64_t* counts, int64_t nranges, void* dst, int64_t dst_rows,
                  int64_t max_threads, int64_t* rows_out) {
  if (rows_out != nullptr) *rows_out = 0;
  EVS_REQUIRE(row_bytes > 0 && nranges >= 0 && max_threads >= 1 && src_rows >= 0 &&
                  dst_rows >= 0 && num_tables >= 0,
              "%s: row_bytes > 0, nranges >= 0, max_threads >= 1 and src_rows, dst_rows, "
              "num_tables >= 0", name);
  EVS_REQUIRE(nranges == 0 || num_tables == 0 ||
                  (srcs != nullptr && dst != nullptr && starts != nullptr && counts != nullptr),
              "%s: null pointer", name);
  for (int64_t j = 0; j < num_tables && nranges > 0; j++)
    EVS_REQUIRE(srcs[j] != nullptr, "%s: table %lld is null", name, static_cast<long long>(j));
  // every range is checked before anything is copied
  std::vector<int64_t> first_row;
  const int rc = check_ranges(name, src_rows, starts, counts, nranges, dst_rows, &first_row);
  if (rc != EVS_OK) return rc;
  const int64_t rows = first_row[nranges];
  if (rows_out != nullptr) *rows_out = rows;  // the copy below cannot fail
  if (rows == 0 || num_tables == 0) return EVS_OK;
  const int64_t total = rows * num_tables;
  const int64_t threads = threads_for(total * row_bytes, max_threads);
  const char* const* s = reinterpret_cast<const char* const*>(srcs);
  char* d = static_cast<char*>(dst);
  if (threads == 1) {
    copy_tables(s, rows, row_bytes, starts, counts, first_row.data(), nranges, d, dst_rows, 0,
                total);
    return EVS_OK;
  }
  const int64_t* fr = first_row.data();
  parallel_for(static_cast<int>(threads), [&](int t) {
    copy_tables(s, rows, row_bytes, starts, counts, fr, nranges, d, dst_rows,
                total * t / threads, total * (t + 1) / threads);
  });
  return EVS_OK;
}

// ---------------------------------------------------------------- delivery into host memory

constexpr int64_t kMinDeliverBytesPerThread = int64_t{2} << 20;

// Copy `nruns` runs of `len` bytes, packed in `src`, to dst at pitch `dst_pitch`: one thread's
// share is packed bytes [b0, b1).
void unpack_runs(char* dst, int64_t dst_pitch, const char* src, int64_t len, int64_t b0,
                 int64_t b1) {
  while (b0 < b1) {
    const int64_t r = b0 / len, o = b0 % len;
    const int64_t take = std::min(len - o, b1 - b0);
    copy_bytes(dst + r * dst_pitch + o, src + b0, static_cast<size_t>(take));
    b0 += take;
  }
  if (EVS_HOST_NT_STORES) stream_fence();
}

void unpack_parallel(char* dst, int64_t dst_pitch, const char* src, int64_t nruns, int64_t len,
                     int64_t max_threads) {
  const int64_t bytes = nruns * len;
  const int64_t threads = threads_for(bytes, max_threads, kMinDeliverBytesPerThread);
  if (threads == 1) {
    unpack_runs(dst, dst_pitch, src, len, 0, bytes);
    return;
  }
  parallel_for(static_cast<int>(threads), [&](int t) {
    // shares start on 64-byte boundaries of the packed bytes
    const int64_t b0 = (bytes * t / threads) & ~int64_t{63};
    const int64_t b1 = t + 1 == threads ? bytes : (bytes * (t + 1) / threads) & ~int64_t{63};
    unpack_runs(dst, dst_pitch, src, len, b0, b1);
  });
}

// One batch of a delivery: runs [run0, run0 + nruns), bytes [offset, offset + len) of each.
struct Batch {
  int64_t run0, nruns, offset, len;
};

// The host copy of the last batch overlaps no copy engine work: it is the delivery's tail. Split
// the last batch into pieces of 1/2, 1/4, 1/8 and 1/8 of it, by runs when it has 8 or more, else by
// bytes within its runs (64-byte multiples), so that all but the last piece overlap a copy. Too
// small a batch is left whole.
constexpr int64_t kMinSplitBytes = int64_t{1} << 20;

void split_last(std::vector<Batch>& batches) {
  if (batches.empty()) return;
  const Batch b = batches.back();
  if (b.nruns * b.len < kMinSplitBytes) return;
  std::vector<Batch> pieces;
  if (b.nruns >= 8) {
    int64_t r = b.run0;
    const int64_t end = b.run0 + b.nruns;
    for (int64_t part : {b.nruns / 2, b.nruns / 4, b.nruns / 8}) {
      pieces.push_back({r, part, b.offset, b.len});
      r += part;
    }
    pieces.push_back({r, end - r, b.offset, b.len});
  } else {
    if (b.len < 8 * 64) return;
    int64_t o = b.offset;
    const int64_t end = b.offset + b.len;
    for (int64_t div : {2, 4, 8}) {
      const int64_t part = (b.len / div) & ~int64_t{63};
      pieces.push_back({b.run0, b.nruns, o, part});
      o += part;
    }
    pieces.push_back({b.run0, b.nruns, o, end - o});
  }
  batches.pop_back();
  batches.insert(batches.end(), pieces.begin(), pieces.end());
}

int deliver(char* dst, int64_t dst_pitch, const char* src, int64_t src_pitch, int64_t runs,
            int64_t run_bytes, char* const bounce[2], int64_t bounce_bytes, int64_t max_threads,
            hipStream_t stream, hipEvent_t ev[2]) {
  std::vector<Batch> batches;
  if (run_bytes <= bounce_bytes) {
    const int64_t per = bounce_bytes / run_bytes;
    for (int64_t r = 0; r < runs; r += per) batches.push_back({r, std::min(per, runs - r), 0, run_bytes});
  } else {
    for (int64_t r = 0; r < runs; r++)
      for (int64_t o = 0; o < run_bytes; o += bounce_bytes)
        batches.push_back({r, 1, o, std::min(bounce_bytes, run_bytes - o)});
  }
  split_last(batches);
  auto issue = [&](size_t i) -> int {
    const Batch& b = batches[i];
    const int rc = copy_runs(bounce[i & 1], b.len, src + b.run0 * src_pitch + b.offset,
                             b.nruns > 1 ? src_pitch : b.len, b.len, b.nruns,
                             hipMemcpyDeviceToHost, stream);
    if (rc != EVS_OK) return rc;
    EVS_HIP(hipEventRecord(ev[i & 1], stream));
    return EVS_OK;
  };
  int rc = issue(0);
  if (rc != EVS_OK) return rc;
  for (size_t i = 0; i < batches.size(); i++) {
    // the other bounce buffer was emptied by the previous iteration's host copy
    if (i + 1 < batches.size() && (rc = issue(i + 1)) != EVS_OK) return rc;
    EVS_HIP(hipEventSynchronize(ev[i & 1]));
    const Batch& b = batches[i];
    unpack_parallel(dst + b.run0 * dst_pitch + b.offset, dst_pitch, bounce[i & 1], b.nruns, b.len,
                    max_threads);
  }
  return EVS_OK;
}

}  // namespace
}  // namespace evs

extern "C" int evs_host_gather_ranges(const void* src, int64_t src_rows, int64_t row_bytes,
                                      const int64_t* starts, const int64_t* counts,
                                      int64_t nranges, void* dst, int64_t dst_rows,
                                      int64_t max_threads, int64_t* rows_out) {
  evs::clear_error();
  const void* srcs[1] = {src};
  return evs::gather_tables("evs_host_gather_ranges", srcs, 1, src_rows, row_bytes, starts,
                            counts, nranges, dst, dst_rows, max_threads, rows_out);
}

extern "C" int evs_host_gather_tables(const void* const* srcs, int64_t num_tables,
                                      int64_t src_rows, int64_t row_bytes, const int64_t* starts,
                                      const int64_t* counts, int64_t nranges, void* dst,
                                      int64_t dst_rows, int64_t max_threads, int64_t* rows_out) {
  evs::clear_error();
  return evs::gather_tables("evs_host_gather_tables", srcs, num_tables, src_rows, row_bytes,
                            starts, counts, nranges, dst, dst_rows, max_threads, rows_out);
}

extern "C" int evs_deliver_rows(void* dst, int64_t dst_pitch, const void* src, int64_t src_pitch,
                                int64_t runs, int64_t run_bytes, void* bounce0, void* bounce1,
                                int64_t bounce_bytes, int64_t max_threads, void* stream) {
  evs::clear_error();
  EVS_REQUIRE(runs >= 0 && run_bytes >= 0 && max_threads >= 1,
              "evs_deliver_rows: runs, run_bytes >= 0 and max_threads >= 1");
  if (runs == 0 || run_bytes == 0) return EVS_OK;
  EVS_REQUIRE(dst != nullptr && src != nullptr && bounce0 != nullptr && bounce1 != nullptr,
              "evs_deliver_rows: null pointer");
  EVS_REQUIRE(bounce0 != bounce1, "evs_deliver_rows: the two bounce buffers must differ");
  EVS_REQUIRE(bounce_bytes >= 64 && bounce_bytes % 64 == 0,
              "evs_deliver_rows: bounce_bytes is a positive multiple of 64, got %lld",
              static_cast<long long>(bounce_bytes));
  EVS_REQUIRE(runs == 1 || (src_pitch >= run_bytes && dst_pitch >= run_bytes),
              "evs_deliver_rows: pitches below the run length (%lld, %lld < %lld)",
              static_cast<long long>(src_pitch), static_cast<long long>(dst_pitch),
              static_cast<long long>(run_bytes));
  hipEvent_t ev[2] = {nullptr, nullptr};
  for (auto& e : ev) EVS_HIP(hipEventCreateWithFlags(&e, hipEventDisableTiming));
  char* const bounce[2] = {static_cast<char*>(bounce0), static_cast<char*>(bounce1)};
  const int rc = evs::deliver(static_cast<char*>(dst), dst_pitch, static_cast<const char*>(src),
                              src_pitch, runs, run_bytes, bounce, bounce_bytes, max_threads,
                              evs::as_stream(stream), ev);
  if (rc != EVS_OK) (void)hipStreamSynchronize(evs::as_stream(stream));  // no copy left behind
  for (auto& e : ev) (void)hipEventDestroy(e);
  return rc;
}
