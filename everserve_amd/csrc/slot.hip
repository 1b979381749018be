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
// for: those of the batch it waits on, and for batches not reached yet, the rows whose first word
// of this thread has not arrived (slot.cu:176-199). A counter after the sequence counters holds
// the workgroups that named; the last to finish clears LATE. When a wait ends without a member,
// that member's missing words are summed as zeros.
//
// The launch is laid out for latency. Wave 0 reads the sequence counter, the order words and the
// buffer table in one round of independent loads, one lane a word, while every thread loads its
// input; the lanes then resolve, per order position, where the member's words are read and (push)
// where this member's go, into LDS. A poll issues the loads of every member of a batch back to
// back from those addresses and waits once, and a batch is every member (up to 8) at 1 or 2 words
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
// covers a whole batch, so a call of k <= 8 members at 1 word a thread (the driver's setting)
// waits for one round trip a poll, not one a batch.
template <int W>
constexpr int batch_of() {
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

__device__ __forceinline__ uint64_t load_sys(const uint64_t* p) {
  return __hip_atomic_load(p, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_SYSTEM);
}

__device__ __forceinline__ void store_sys(uint64_t* p, uint64_t v) {
  __hip_atomic_store(p, v, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_SYSTEM);
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

template <int W, bool kPush>
__global__ __launch_bounds__(kSlotThreads) void slot_all_reduce(SlotArgs a) {
  constexpr int kBatch = batch_of<W>();
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

  // publish this member's words
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

  float lo[W], hi[W];
  uint32_t valid = 0;
#pragma unroll
  for (int j = 0; j < W; j++) {
    lo[j] = 0.f;
    hi[j] = 0.f;
    if (b0 + j * kSlotThreads < a.n2) valid |= 1u << j;
  }
  const bool watch = threadIdx.x == 0;
  const int64_t t0 = wall_clock64();
  bool counted = false;
  bool released = false;  // by ABORT or the timeout: later batches are not waited for
  uint32_t polls = 0;
  uint64_t* late_count = reinterpret_cast<uint64_t*>(a.seqs + a.late_index);

  for (int b = 0; b < nmem; b += kBatch) {
    const uint64_t* src[kBatch];
    int ms[kBatch];
    const int nm = nmem - b < kBatch ? nmem - b : kBatch;
    uint64_t w[kBatch][W];
    uint32_t todo[kBatch];
#pragma unroll
    for (int q = 0; q < kBatch; q++) {
      src[q] = q < nm ? uniform_ptr(s_src[b + q]) : nullptr;
      ms[q] = q < nm ? __builtin_amdgcn_readfirstlane(s_row[b + q]) : -1;
      todo[q] = (src[q] != nullptr && !released) ? valid : 0u;
#pragma unroll
      for (int j = 0; j < W; j++) w[q][j] = 0ull;
    }
    while (true) {
#pragma unroll
      for (int q = 0; q < kBatch; q++) {
        if (!todo[q]) continue;
#pragma unroll
        for (int j = 0; j < W; j++)
          if (todo[q] >> j & 1) w[q][j] = load_sys(src[q] + b0 + j * kSlotThreads);
      }
      uint32_t any = 0;
#pragma unroll
      for (int q = 0; q < kBatch; q++) {
#pragma unroll
        for (int j = 0; j < W; j++)
          if ((todo[q] >> j & 1) && static_cast<uint32_t>(w[q][j] >> 32) == seq)
            todo[q] &= ~(1u << j);
        any |= todo[q];
      }
      if (!any) break;
      if ((++polls % kCheckEvery) == 0) {
        const int64_t waited = wall_clock64() - t0;
        const uint64_t* c = reinterpret_cast<const uint64_t*>(a.ctrl);
        if (load_sys(c + EVS_ABORT) != 0 || waited > a.timeout_ticks) {
          released = true;
          break;
        }
        if (watch) {
          const int64_t bound = static_cast<int64_t>(load_sys(c + EVS_BOUND));
          if (bound > 0 && waited * 1000000 / a.clock_khz > bound) {
            // the rows of this batch it still waits on, and of the batches after it, the rows
            // whose first word of this thread has not arrived
            int64_t late = 0;
#pragma unroll
            for (int q = 0; q < kBatch; q++)
              if (todo[q]) late |= int64_t{1} << ms[q];
            for (int q = b + nm; q < nmem; q++) {
              const uint64_t* p = s_src[q];
              if (p == nullptr) continue;
              if (static_cast<uint32_t>(load_sys(p + b0) >> 32) != seq)
                late |= int64_t{1} << s_row[q];
            }
            if (!counted) {
              __hip_atomic_fetch_add(late_count, uint64_t{1}, __ATOMIC_RELAXED,
                                     __HIP_MEMORY_SCOPE_AGENT);
              counted = true;
            }
            store_sys(reinterpret_cast<uint64_t*>(a.ctrl + EVS_LATE), static_cast<uint64_t>(late));
          }
        }
      }
      __builtin_amdgcn_s_sleep(1);
    }
    // sum the batch in order; a word that never arrived, or a row out of range, counts as zero
#pragma unroll
    for (int q = 0; q < kBatch; q++) {
      if (q >= nm) continue;
#pragma unroll
      for (int j = 0; j < W; j++) {
        const uint32_t v = (todo[q] >> j & 1) || ms[q] < 0 ? 0u : static_cast<uint32_t>(w[q][j]);
        lo[j] += __uint_as_float((v & 0xffffu) << 16);
        hi[j] += __uint_as_float(v & 0xffff0000u);
      }
    }
  }
  // the wait is over; the last workgroup that named clears the word
  if (counted && __hip_atomic_fetch_add(late_count, ~uint64_t{0}, __ATOMIC_RELAXED,
                                        __HIP_MEMORY_SCOPE_AGENT) == 1)
    store_sys(reinterpret_cast<uint64_t*>(a.ctrl + EVS_LATE), 0);
#pragma unroll
  for (int j = 0; j < W; j++) {
    const int i = b0 + j * kSlotThreads;
    if (i < a.n2) a.out[i] = to_bf16(lo[j]) | (to_bf16(hi[j]) << 16);
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
