// The slot collective's kernel, on gfx950: a decode-size bf16 all-reduce over LL words that a HIP
// graph can capture, the drop-in for core/csrc/slot.cu:72-281 behind the same arguments.
//
// A word is 8 bytes: the call's sequence number in the high 32 bits and two bf16 values in the low
// 32, written with one 64-bit store, so a reader that sees the number sees the data. Each member
// publishes its words, then waits until every listed member's words carry the number, then sums
// the members in the listed order in fp32 from 0.0f and rounds once to bf16 (torch's rule; NaN
// becomes 0x7FC0). Where the words go is the variant's:
//
//   pull: each member's buffer is [2 parities][maxn/2] words; a member writes its own buffer
//         and reads every member's;
//   push: each member's buffer is [2 parities][8 senders][maxn/2] words; a member writes its
//         words into every member's buffer at its own sender index and reads only its own buffer.
//
// The member order, the buffer table and the per-workgroup sequence counters live in device
// memory and are read on every launch, so a captured graph follows a change of members or buffers
// without recapture. The parity of the number picks the half of a buffer, so two back-to-back
// calls never overwrite words a slower member still reads.
//
// Waiting is bounded twice. Every 1024 polls a thread reads the member's ABORT control word
// (core/csrc/slot.cu:174-175) and the wall clock; past `timeout_ns` it stops waiting by itself.
// Thread 0 of each workgroup, past the BOUND word (ns), writes into LATE the rows it still waits
// for: those of the group of members it waits on, and for groups not reached yet, the rows whose
// first word of this thread has not arrived (slot.cu:176-199). A counter after the sequence
// counters holds the workgroups that named; the last to finish clears LATE. When a wait ends
// without a member, that member's missing words are summed as zeros.
//
// The launch is laid out for latency. Wave 0 reads the sequence counter, the order words and the
// buffer table in one round of independent loads, one lane a word, while every thread loads its
// input; the lanes then resolve, per order position, where the member's words are read and (push)
// where this member's go, into LDS. A poll issues the loads of every member of a group back to
// back from those addresses and waits once, and a group is every member (up to 8) at 1 or 2 words
// a thread, so a call of 8 members waits for one round trip a poll, not one per member.

#include "common.hpp"

namespace evs {

int wall_clock_khz(int64_t* khz);  // reduce.hip

namespace {

constexpr int kSlotThreads = 256;
constexpr int kMaxRows = EVS_MAX_ROWS;
constexpr uint32_t kCheckEvery = 1024;

// Members whose words a thread waits on together: every member (up to 8) at 1 or 2 words a
// thread, 4 at more, where 8 members' words would hold 64-256 VGPRs. One round of loads then
// covers a whole group, so a call of k <= 8 members at 1 word a thread (the driver's setting)
// waits for one round trip a poll, not one a member.
template <int W>
constexpr int group_of() {
  return W <= 2 ? kMaxRows : 4;
}

struct SlotArgs {
  const uint32_t* x;        // the member's input, as pairs of bf16
  uint32_t* out;
  int n2;                   // pairs
  const int64_t* bufs;      // device table: each row's word buffer
  int64_t* ctrl;            // the member's control row (EVS_CTRL_WORDS words)
  const int32_t* order;     // device [count, rows...]
  int64_t* seqs;            // device: a counter per workgroup, then the named-workgroup count
  int64_t late_index;       // where that count sits in seqs
  int my;
  int64_t maxn2;
  int64_t timeout_ticks;
  int64_t clock_khz;
};

// Every word these kernels read or write at system scope is global memory (device memory, or host
// memory mapped for the device), so the accesses go through global_ rather than flat_
// instructions: a flat store might alias LDS, and the compiler then waits for every such store to
// complete before the next LDS read (which held each call's first poll behind its publish).
typedef __attribute__((address_space(1))) uint64_t global_u64;

__device__ __forceinline__ uint64_t load_sys(const uint64_t* p) {
  return __hip_atomic_load((const global_u64*)(p), __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_SYSTEM);
}

__device__ __forceinline__ void store_sys(uint64_t* p, uint64_t v) {
  __hip_atomic_store((global_u64*)(p), v, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_SYSTEM);
}

// A value the same in every lane, moved to scalar registers.
template <typename T>
__device__ __forceinline__ T* uniform_ptr(T* p) {
  const uint64_t v = reinterpret_cast<uint64_t>(p);
  const uint32_t lo = __builtin_amdgcn_readfirstlane(static_cast<uint32_t>(v));
  const uint32_t hi = __builtin_amdgcn_readfirstlane(static_cast<uint32_t>(v >> 32));
  return reinterpret_cast<T*>((static_cast<uint64_t>(hi) << 32) | lo);
}

__device__ __forceinline__ uint32_t to_bf16(float f) {
  const uint32_t u = __float_as_uint(f);
  if ((u & 0x7fffffffu) > 0x7f800000u) return 0x7fc0u;
  return (u + 0x7fffu + ((u >> 16) & 1u)) >> 16;
}

// The words one thread reads for a group of up to G members of the order: word[q][j] is word j
// of the group's q-th member (its buffer at src[q], its row row[q]); bit j of pending[q] stays set
// until that word carries this call's number.
template <int W, int G>
struct Group {
  int size;
  const uint64_t* src[G];
  int row[G];
  uint64_t word[G][W];
  uint32_t pending[G];
};

// One poll: every pending word of the group is loaded (all loads issued before any is tested),
// and those that now carry `seq` stop pending. Returns whether any word still pends.
template <int W, int G>
__device__ __forceinline__ bool read_pending(Group<W, G>& g, int b0, uint32_t seq) {
#pragma unroll
  for (int q = 0; q < G; q++) {
    if (g.pending[q] == 0) continue;
#pragma unroll
    for (int j = 0; j < W; j++)
      if ((g.pending[q] >> j) & 1u) g.word[q][j] = load_sys(g.src[q] + b0 + j * kSlotThreads);
  }
  uint32_t still = 0;
#pragma unroll
  for (int q = 0; q < G; q++) {
#pragma unroll
    for (int j = 0; j < W; j++) {
      const bool arrived = static_cast<uint32_t>(g.word[q][j] >> 32) == seq;
      if (arrived) g.pending[q] &= ~(1u << j);
    }
    still |= g.pending[q];
  }
  return still != 0;
}

// The group's words added into the running sums, member after member in the group's order. A word
// still pending (its member never came) adds +0.0, which changes no sum that started at +0.0.
template <int W, int G>
__device__ __forceinline__ void add_in_order(const Group<W, G>& g, float (&sum_lo)[W],
                                             float (&sum_hi)[W]) {
#pragma unroll
  for (int q = 0; q < G; q++) {
    if (q >= g.size) continue;
#pragma unroll
    for (int j = 0; j < W; j++) {
      const bool use = ((g.pending[q] >> j) & 1u) == 0 && g.row[q] >= 0;
      const uint32_t pair = use ? static_cast<uint32_t>(g.word[q][j]) : 0u;
      sum_lo[j] += __uint_as_float(pair << 16);            // the low bf16, widened
      sum_hi[j] += __uint_as_float(pair & 0xffff0000u);    // the high bf16, in place
    }
  }
}

// One thread's bounded wait over the whole call: when it started, the polls so far, whether it
// gave up (ABORT or the timeout: later groups are then not waited for), and whether this
// workgroup has named late rows (counted once in `namers`, the word after the sequence counters).
struct Waiter {
  int64_t start;
  uint32_t polls;
  bool gave_up;
  bool named;
  uint64_t* namers;

  // Called after a poll that left words pending: false when the wait is over. Every kCheckEvery
  // polls it reads ABORT and the clock; thread 0, past BOUND, also writes the rows it still
  // waits for into LATE.
  template <int W, int G>
  __device__ __forceinline__ bool may_go_on(const SlotArgs& a, const Group<W, G>& g,
                                            const uint64_t* const (&src_at)[kMaxRows],
                                            const int (&row_at)[kMaxRows], int later, int b0,
                                            uint32_t seq) {
    if (++polls % kCheckEvery != 0) return true;
    const int64_t waited = wall_clock64() - start;
    const uint64_t* ctrl = reinterpret_cast<const uint64_t*>(a.ctrl);
    if (load_sys(ctrl + EVS_ABORT) != 0 || waited > a.timeout_ticks) {
      gave_up = true;
      return false;
    }
    if (threadIdx.x == 0) {
      const int64_t bound_ns = static_cast<int64_t>(load_sys(ctrl + EVS_BOUND));
      if (bound_ns > 0 && waited * 1000000 / a.clock_khz > bound_ns)
        name_late(a, late_rows(g, src_at, row_at, later, b0, seq));
    }
    return true;
  }

  // The rows this thread still waits for: in the current group, each member with a word pending;
  // of the members in groups not reached yet (order positions from `later` on; an unlisted
  // position has no address), each whose first word of this thread does not carry `seq`
  // (core/csrc/slot.cu:176-199 names the same rows).
  template <int W, int G>
  __device__ __forceinline__ static int64_t late_rows(const Group<W, G>& g,
                                                      const uint64_t* const (&src_at)[kMaxRows],
                                                      const int (&row_at)[kMaxRows], int later,
                                                      int b0, uint32_t seq) {
    int64_t rows = 0;
#pragma unroll
    for (int q = 0; q < G; q++)
      if (g.pending[q] != 0) rows |= int64_t{1} << g.row[q];
#pragma unroll
    for (int m = 0; m < kMaxRows; m++) {
      if (m < later || src_at[m] == nullptr) continue;
      if (static_cast<uint32_t>(load_sys(src_at[m] + b0) >> 32) != seq)
        rows |= int64_t{1} << row_at[m];
    }
    return rows;
  }

  // Write LATE, counting this workgroup among the namers the first time. LATE is written at every
  // check, since another workgroup's clear may have raced this one's earlier write.
  __device__ __forceinline__ void name_late(const SlotArgs& a, int64_t rows) {
    if (!named) {
      __hip_atomic_fetch_add(namers, uint64_t{1}, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
      named = true;
    }
    store_sys(reinterpret_cast<uint64_t*>(a.ctrl + EVS_LATE), static_cast<uint64_t>(rows));
  }

  // The wait is over: the last namer to get here clears LATE.
  __device__ __forceinline__ void done(const SlotArgs& a) {
    if (named && __hip_atomic_fetch_add(namers, ~uint64_t{0}, __ATOMIC_RELAXED,
                                        __HIP_MEMORY_SCOPE_AGENT) == 1)
      store_sys(reinterpret_cast<uint64_t*>(a.ctrl + EVS_LATE), 0);
  }
};

template <int W, bool kPush>
__global__ __launch_bounds__(kSlotThreads) void slot_all_reduce(SlotArgs a) {
  constexpr int kGroup = group_of<W>();
  // per order position q: the words this member reads (member q's, this call's parity half) and,
  // for push, where it writes its own into member q's buffer; null for a row out of range
  __shared__ const uint64_t* s_src[kMaxRows];
  __shared__ uint64_t* s_dst[kMaxRows];
  __shared__ uint64_t* s_mine;  // pull: this member's own half, where it publishes
  __shared__ int s_row[kMaxRows];
  __shared__ uint32_t s_seq;
  __shared__ int s_n;

  const int b0 = blockIdx.x * W * kSlotThreads + threadIdx.x;
  // the input, read before the prologue's loads return: nothing it depends on is pending
  uint32_t xin[W];
#pragma unroll
  for (int j = 0; j < W; j++) {
    const int i = b0 + j * kSlotThreads;
    xin[j] = i < a.n2 ? a.x[i] : 0u;
  }

  if (threadIdx.x < 64) {
    // One round of independent loads, one lane a word: this workgroup's sequence counter, the
    // order words and the buffer table.
    const int lane = threadIdx.x;
    const int64_t prev =
        lane == 0 ? static_cast<int64_t>(__hip_atomic_load(
                        reinterpret_cast<const uint64_t*>(a.seqs + blockIdx.x), __ATOMIC_RELAXED,
                        __HIP_MEMORY_SCOPE_AGENT))
                  : 0;
    const int o = lane <= kMaxRows ? a.order[lane] : 0;
    const int64_t buf = lane < kMaxRows ? a.bufs[lane] : 0;
    const int64_t s = __shfl(prev, 0) + 1;
    if (lane == 0) a.seqs[blockIdx.x] = s;
    const uint32_t seq = static_cast<uint32_t>(s);
    const size_t parity_off = static_cast<size_t>(seq & 1u) * static_cast<size_t>(a.maxn2);
    int n = __shfl(o, 0);
    n = n < 0 ? 0 : (n > kMaxRows ? kMaxRows : n);
    // lane q < n stands for order position q; a row out of range is never waited for
    const int r = __shfl(o, (lane + 1) & 63);
    const bool valid = lane < n && r >= 0 && r < kMaxRows;
    const int64_t their = __shfl(buf, valid ? r : 0);
    const int64_t mine = __shfl(buf, a.my);
    if (lane < kMaxRows) {
      const uint64_t* src =
          kPush ? reinterpret_cast<const uint64_t*>(mine) + parity_off * kMaxRows +
                      static_cast<size_t>(r) * a.maxn2
                : reinterpret_cast<const uint64_t*>(their) + parity_off;
      s_src[lane] = valid ? src : nullptr;
      s_dst[lane] = valid && kPush ? reinterpret_cast<uint64_t*>(their) + parity_off * kMaxRows +
                                         static_cast<size_t>(a.my) * a.maxn2
                               : nullptr;
      s_row[lane] = valid ? r : -1;
    }
    if (lane == 0) {
      s_seq = seq;
      s_n = n;
      s_mine = reinterpret_cast<uint64_t*>(mine) + parity_off;
    }
  }
  __syncthreads();
  const uint32_t seq = s_seq;
  const int nmem = s_n;
  const uint64_t tag = static_cast<uint64_t>(seq) << 32;
  // Every order position's read address and row, out of LDS into scalar registers once, before
  // the first store: an LDS read behind outstanding stores may have to wait for them.
  const uint64_t* src_at[kMaxRows];
  int row_at[kMaxRows];
#pragma unroll
  for (int q = 0; q < kMaxRows; q++) {
    src_at[q] = q < nmem ? uniform_ptr(s_src[q]) : nullptr;
    row_at[q] = q < nmem ? __builtin_amdgcn_readfirstlane(s_row[q]) : -1;
  }

  // publish this member's words (push: into every member's buffer, one member at a time)
  if (kPush) {
    for (int q = 0; q < nmem; q++) {
      uint64_t* dst = uniform_ptr(s_dst[q]);
      if (dst == nullptr) continue;
#pragma unroll
      for (int j = 0; j < W; j++) {
        const int i = b0 + j * kSlotThreads;
        if (i < a.n2) store_sys(dst + i, tag | xin[j]);
      }
    }
  } else {
    uint64_t* mine = uniform_ptr(s_mine);
#pragma unroll
    for (int j = 0; j < W; j++) {
      const int i = b0 + j * kSlotThreads;
      if (i < a.n2) store_sys(mine + i, tag | xin[j]);
    }
  }

  // Members are taken in the listed order, a group of up to kGroup at a time: the group's words
  // are read until they all carry this call's number (or the wait is given up), then added into
  // the running sums. Bit j of `owned` is set when this thread has a word j.
  uint32_t owned = 0;
  float sum_lo[W], sum_hi[W];  // running fp32 sums of each word's low and high bf16
#pragma unroll
  for (int j = 0; j < W; j++) {
    sum_lo[j] = sum_hi[j] = 0.f;
    if (b0 + j * kSlotThreads < a.n2) owned |= 1u << j;
  }
  Waiter waiter{wall_clock64(), 0u, false, false,
                reinterpret_cast<uint64_t*>(a.seqs + a.late_index)};
#pragma unroll
  for (int first = 0; first < kMaxRows; first += kGroup) {  // unrolled: every index is static
    if (first >= nmem) break;
    Group<W, kGroup> g;
    g.size = nmem - first < kGroup ? nmem - first : kGroup;
#pragma unroll
    for (int q = 0; q < kGroup; q++) {
      g.src[q] = src_at[first + q];
      g.row[q] = row_at[first + q];
      g.pending[q] = g.src[q] != nullptr && !waiter.gave_up ? owned : 0u;
#pragma unroll
      for (int j = 0; j < W; j++) g.word[q][j] = 0ull;  // a word never read adds +0.0
    }
    while (read_pending(g, b0, seq)) {
      if (!waiter.may_go_on(a, g, src_at, row_at, first + kGroup, b0, seq)) break;
      __builtin_amdgcn_s_sleep(1);
    }
    add_in_order(g, sum_lo, sum_hi);
  }
  waiter.done(a);
#pragma unroll
  for (int j = 0; j < W; j++) {
    const int i = b0 + j * kSlotThreads;
    if (i < a.n2) a.out[i] = to_bf16(sum_lo[j]) | (to_bf16(sum_hi[j]) << 16);
  }
}

template <bool kPush>
void launch(int words, unsigned blocks, hipStream_t s, const SlotArgs& a) {
  switch (words) {
    case 16: hipLaunchKernelGGL((slot_all_reduce<16, kPush>), dim3(blocks), dim3(kSlotThreads), 0, s, a); break;
    case 8: hipLaunchKernelGGL((slot_all_reduce<8, kPush>), dim3(blocks), dim3(kSlotThreads), 0, s, a); break;
    case 4: hipLaunchKernelGGL((slot_all_reduce<4, kPush>), dim3(blocks), dim3(kSlotThreads), 0, s, a); break;
    case 2: hipLaunchKernelGGL((slot_all_reduce<2, kPush>), dim3(blocks), dim3(kSlotThreads), 0, s, a); break;
    default: hipLaunchKernelGGL((slot_all_reduce<1, kPush>), dim3(blocks), dim3(kSlotThreads), 0, s, a); break;
  }
}

}  // namespace
}  // namespace evs

extern "C" int evs_slot_all_reduce(const void* inp, void* out, int64_t n, const int64_t* bufs,
                                   int64_t* ctrl, const int32_t* order, int64_t* seqs,
                                   int64_t num_seqs, int64_t row, int64_t maxn, int64_t words,
                                   int push, int64_t timeout_ns, void* stream) {
  evs::clear_error();
  EVS_REQUIRE(words == 1 || words == 2 || words == 4 || words == 8 || words == 16,
              "evs_slot_all_reduce: words per thread must be 1, 2, 4, 8 or 16");
  EVS_REQUIRE(n >= 0 && n % 2 == 0 && n <= maxn,
              "evs_slot_all_reduce: an even element count up to %lld", static_cast<long long>(maxn));
  EVS_REQUIRE(maxn >= 2 && maxn % 2 == 0 && maxn / 2 < (int64_t{1} << 31),
              "evs_slot_all_reduce: maxn must be even and below 2^32");
  EVS_REQUIRE(row >= 0 && row < EVS_MAX_ROWS, "evs_slot_all_reduce: row out of range");
  const int64_t one_word_blocks = (maxn / 2 + 255) / 256;  // slot_blocks(maxn, 1)
  EVS_REQUIRE(num_seqs > one_word_blocks, "evs_slot_all_reduce: too few counters (%lld, need %lld)",
              static_cast<long long>(num_seqs), static_cast<long long>(one_word_blocks + 1));
  if (n == 0) return EVS_OK;
  EVS_REQUIRE(inp != nullptr && out != nullptr && bufs != nullptr && ctrl != nullptr &&
                  order != nullptr && seqs != nullptr,
              "evs_slot_all_reduce: null pointer");
  EVS_REQUIRE((reinterpret_cast<int64_t>(inp) & 3) == 0 && (reinterpret_cast<int64_t>(out) & 3) == 0,
              "evs_slot_all_reduce: input and output must be 4-byte aligned");
  int64_t khz = 0;
  const int rc = evs::wall_clock_khz(&khz);
  if (rc != EVS_OK) return rc;
  if (timeout_ns <= 0) timeout_ns = int64_t{30} * 1000000000;
  evs::SlotArgs a{};
  a.x = static_cast<const uint32_t*>(inp);
  a.out = static_cast<uint32_t*>(out);
  a.n2 = static_cast<int>(n / 2);
  a.bufs = bufs;
  a.ctrl = ctrl + row * EVS_CTRL_WORDS;
  a.order = order;
  a.seqs = seqs;
  a.late_index = one_word_blocks;
  a.my = static_cast<int>(row);
  a.maxn2 = maxn / 2;
  a.timeout_ticks = timeout_ns / 1000 * khz / 1000;
  a.clock_khz = khz;
  const int64_t per_block = int64_t{evs::kSlotThreads} * words;
  const unsigned blocks = static_cast<unsigned>((n / 2 + per_block - 1) / per_block);
  if (push)
    evs::launch<true>(static_cast<int>(words), blocks, evs::as_stream(stream), a);
  else
    evs::launch<false>(static_cast<int>(words), blocks, evs::as_stream(stream), a);
  EVS_LAUNCHED("evs_slot_all_reduce");
  return EVS_OK;
}
