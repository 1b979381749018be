// The node store's commit copy, on the host: a staged step's rows into the per-(layer, head)
// tables, with each written row's step and CRC32C (store/src/storage.rs:864-957, the copy loop
// :916-943; Layer::mark_written :494-504). The store itself is the reference's Rust service; this
// is the same copy as a library call, for a store that runs in this process or links this
// library, and what the restore reads back (the written steps and the checksums) is laid out as
// the Rust store keeps it (written_step and crc per slot, storage.rs:364-376).
//
// CRC32C is the Castagnoli CRC (reflected polynomial 0x82F63B78, initial value and final xor
// 0xFFFFFFFF) the Rust store computes with the crc32c crate. On x86 hosts with SSE4.2 it runs on
// the crc32 instruction, four rows at a time so that the instruction's latency is hidden behind
// three other rows (the rows are independent); elsewhere a byte table.

#include <algorithm>
#include <cstring>
#include <vector>

#include "common.hpp"
#include "host_copy.hpp"
#include "workers.hpp"

// Steps of at least this many bytes write their table rows with nontemporal stores (see
// commit_table); smaller ones with memcpy. On the MI355X box's host, a C2 step (256 MiB over 32
// tables) committed at 55 GB/s on 16 threads with them and 38.7 without, and a 64-slot decode
// step (1 MiB) in 40 us with them and 30 without (the fence and the partial write-combining
// lines cost more than the cache misses save at that size).
#ifndef EVS_STORE_NT_MIN_BYTES
#define EVS_STORE_NT_MIN_BYTES (int64_t{4} << 20)
#endif
// Tables are committed on several threads only when each gets at least this many bytes.
#ifndef EVS_STORE_MIN_BYTES_PER_THREAD
#define EVS_STORE_MIN_BYTES_PER_THREAD (int64_t{128} << 10)
#endif

namespace evs {
namespace {

constexpr uint32_t kCastagnoli = 0x82F63B78u;  // reflected 0x1EDC6F41

struct CrcTable {
  uint32_t t[256];
  CrcTable() {
    for (uint32_t i = 0; i < 256; i++) {
      uint32_t c = i;
      for (int k = 0; k < 8; k++) c = (c >> 1) ^ ((c & 1u) ? kCastagnoli : 0u);
      t[i] = c;
    }
  }
};

const CrcTable& crc_table() {
  static const CrcTable table;
  return table;
}

uint32_t crc_bytes_table(uint32_t c, const uint8_t* p, size_t n) {
  const uint32_t* t = crc_table().t;
  for (size_t i = 0; i < n; i++) c = t[(c ^ p[i]) & 0xffu] ^ (c >> 8);
  return c;
}

#if defined(__x86_64__)
__attribute__((target("sse4.2"))) uint32_t crc_bytes_hw(uint32_t c, const uint8_t* p, size_t n) {
  uint64_t c64 = c;
  size_t i = 0;
  for (; i + 8 <= n; i += 8) {
    uint64_t w;
    std::memcpy(&w, p + i, 8);
    c64 = __builtin_ia32_crc32di(c64, w);
  }
  uint32_t c32 = static_cast<uint32_t>(c64);
  for (; i < n; i++) c32 = __builtin_ia32_crc32qi(c32, p[i]);
  return c32;
}

// Four rows of `bytes` each at once: four independent chains keep the crc32 unit busy.
__attribute__((target("sse4.2"))) void crc_four_hw(const uint8_t* const p[4], size_t bytes,
                                                   uint32_t out[4]) {
  uint64_t c0 = 0xffffffffu, c1 = 0xffffffffu, c2 = 0xffffffffu, c3 = 0xffffffffu;
  size_t i = 0;
  for (; i + 8 <= bytes; i += 8) {
    uint64_t w0, w1, w2, w3;
    std::memcpy(&w0, p[0] + i, 8);
    std::memcpy(&w1, p[1] + i, 8);
    std::memcpy(&w2, p[2] + i, 8);
    std::memcpy(&w3, p[3] + i, 8);
    c0 = __builtin_ia32_crc32di(c0, w0);
    c1 = __builtin_ia32_crc32di(c1, w1);
    c2 = __builtin_ia32_crc32di(c2, w2);
    c3 = __builtin_ia32_crc32di(c3, w3);
  }
  uint32_t c[4] = {static_cast<uint32_t>(c0), static_cast<uint32_t>(c1),
                   static_cast<uint32_t>(c2), static_cast<uint32_t>(c3)};
  for (int r = 0; r < 4; r++) {
    for (size_t j = i; j < bytes; j++) c[r] = __builtin_ia32_crc32qi(c[r], p[r][j]);
    out[r] = ~c[r];
  }
}

bool have_hw_crc() {
  static const bool yes = __builtin_cpu_supports("sse4.2");
  return yes;
}
#else
bool have_hw_crc() { return false; }
#endif

uint32_t crc32c(const uint8_t* p, size_t n) {
#if defined(__x86_64__)
  if (have_hw_crc()) return ~crc_bytes_hw(0xffffffffu, p, n);
#endif
  return ~crc_bytes_table(0xffffffffu, p, n);
}

// CRC32C of `count` rows of `bytes`, row r at rows[r] (pointers), into out[r].
void crc_rows(const uint8_t* const* rows, int64_t count, size_t bytes, uint32_t* out) {
  int64_t r = 0;
#if defined(__x86_64__)
  if (have_hw_crc()) {
    for (; r + 4 <= count; r += 4) crc_four_hw(rows + r, bytes, out + r);
  }
#endif
  for (; r < count; r++) out[r] = crc32c(rows[r], bytes);
}

// One table's commit. Each run of consecutive slots is checksummed from the staged rows (the bytes
// it writes), four rows at a time, then copied, with nontemporal stores when `nt`: a large step's
// slots lie at random places in gigabytes of tables, so a plain store would first miss on every
// line it writes, where the staged rows are read in order. Runs go in order, so a slot named twice
// keeps the last write's rows, step and checksum, as the store's mark after each copy does.
// Returns the slots written for the first time; with `nt` the caller fences the stores.
int64_t commit_table(const uint8_t* staged, uint8_t* table, uint64_t* written_step, uint32_t* crc,
                     int64_t row_bytes, const int64_t* slots, int64_t n, uint64_t step, bool nt) {
  const size_t rb = static_cast<size_t>(row_bytes);
  const uint64_t mark = step > 0 ? step : 1;  // step 0 still counts as written
  int64_t fresh = 0;
  constexpr int64_t kBatch = 64;
  const uint8_t* rows[kBatch];
  uint32_t sums[kBatch];
  int64_t i = 0;
  while (i < n) {
    const int64_t s = slots[i];
    if (s < 0) {  // padding
      i++;
      continue;
    }
    int64_t run = 1;
    while (i + run < n && slots[i + run] == s + run) run++;
    const uint8_t* src = staged + static_cast<size_t>(i) * rb;
    for (int64_t r0 = 0; r0 < run; r0 += kBatch) {
      const int64_t m = std::min(kBatch, run - r0);
      for (int64_t k = 0; k < m; k++) rows[k] = src + static_cast<size_t>(r0 + k) * rb;
      crc_rows(rows, m, rb, sums);
      for (int64_t k = 0; k < m; k++) {
        const int64_t slot = s + r0 + k;
        if (written_step[slot] == 0) fresh++;
        written_step[slot] = mark;
        crc[slot] = sums[k];
      }
    }
    if (nt)
      stream_copy(reinterpret_cast<char*>(table + static_cast<size_t>(s) * rb),
                  reinterpret_cast<const char*>(src), static_cast<size_t>(run) * rb);
    else
      std::memcpy(table + static_cast<size_t>(s) * rb, src, static_cast<size_t>(run) * rb);
    i += run;
  }
  return fresh;
}

constexpr int64_t kMinBytesPerThread = EVS_STORE_MIN_BYTES_PER_THREAD;

}  // namespace
}  // namespace evs

extern "C" int evs_crc32c(const void* data, int64_t bytes, uint32_t* out) {
  evs::clear_error();
  EVS_REQUIRE(out != nullptr && bytes >= 0 && (bytes == 0 || data != nullptr),
              "evs_crc32c: null pointer or negative size");
  *out = evs::crc32c(static_cast<const uint8_t*>(data), static_cast<size_t>(bytes));
  return EVS_OK;
}

extern "C" int evs_crc32c_rows(const void* data, int64_t row_bytes, int64_t rows,
                               uint32_t* out) {
  evs::clear_error();
  EVS_REQUIRE(row_bytes > 0 && rows >= 0, "evs_crc32c_rows: row_bytes > 0 and rows >= 0");
  EVS_REQUIRE(rows == 0 || (data != nullptr && out != nullptr), "evs_crc32c_rows: null pointer");
  const uint8_t* base = static_cast<const uint8_t*>(data);
  constexpr int64_t kBatch = 256;
  const uint8_t* ptrs[kBatch];
  for (int64_t r0 = 0; r0 < rows; r0 += kBatch) {
    const int64_t m = std::min(kBatch, rows - r0);
    for (int64_t k = 0; k < m; k++) ptrs[k] = base + (r0 + k) * row_bytes;
    evs::crc_rows(ptrs, m, static_cast<size_t>(row_bytes), out + r0);
  }
  return EVS_OK;
}

extern "C" int evs_store_commit(const void* stage, int64_t stage_bytes,
                                const int64_t* stage_offsets, int64_t ntables,
                                void* const* tables, uint64_t* const* written_step,
                                uint32_t* const* crc, int64_t num_slots, int64_t row_bytes,
                                const int64_t* slots, int64_t nslots, uint64_t step,
                                int64_t max_threads, int64_t* newly_written) {
  evs::clear_error();
  EVS_REQUIRE(ntables >= 0 && nslots >= 0 && num_slots >= 0 && row_bytes > 0 &&
                  stage_bytes >= 0 && max_threads >= 1,
              "evs_store_commit: negative count, row_bytes <= 0 or max_threads < 1");
  if (newly_written != nullptr) *newly_written = 0;
  if (ntables == 0 || nslots == 0) return EVS_OK;
  EVS_REQUIRE(stage != nullptr && stage_offsets != nullptr && tables != nullptr &&
                  written_step != nullptr && crc != nullptr && slots != nullptr,
              "evs_store_commit: null pointer");
  // everything is checked before anything is written, as the store validates a descriptor first
  // (storage.rs:960-1010)
  for (int64_t i = 0; i < nslots; i++)
    EVS_REQUIRE(slots[i] < num_slots, "evs_store_commit: slot %lld outside 0..%lld",
                static_cast<long long>(slots[i]), static_cast<long long>(num_slots));
  const int64_t span = nslots * row_bytes;
  for (int64_t k = 0; k < ntables; k++) {
    EVS_REQUIRE(stage_offsets[k] >= 0 && stage_offsets[k] <= stage_bytes - span,
                "evs_store_commit: table %lld's rows lie outside the staging bytes",
                static_cast<long long>(k));
    EVS_REQUIRE(tables[k] != nullptr && written_step[k] != nullptr && crc[k] != nullptr,
                "evs_store_commit: table %lld has a null buffer", static_cast<long long>(k));
  }
  const uint8_t* st = static_cast<const uint8_t*>(stage);
  std::vector<int64_t> fresh(static_cast<size_t>(ntables), 0);
  const bool nt = ntables * span >= EVS_STORE_NT_MIN_BYTES;
  auto one = [&](int64_t k) {
    fresh[static_cast<size_t>(k)] =
        evs::commit_table(st + stage_offsets[k], static_cast<uint8_t*>(tables[k]),
                          written_step[k], crc[k], row_bytes, slots, nslots, step, nt);
    if (nt) evs::stream_fence();  // this thread's rows are in memory before the commit returns
  };
  int64_t threads = std::min(max_threads, ntables);
  threads = std::min(threads, std::max<int64_t>(1, ntables * span / evs::kMinBytesPerThread));
  if (threads <= 1) {
    for (int64_t k = 0; k < ntables; k++) one(k);
  } else {
    evs::parallel_for(static_cast<int>(threads), [&](int t) {
      for (int64_t k = t; k < ntables; k += threads) one(k);
    });
  }
  if (newly_written != nullptr) {
    int64_t total = 0;
    for (int64_t f : fresh) total += f;
    *newly_written = total;
  }
  return EVS_OK;
}
