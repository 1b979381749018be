// The reduction stage of the failure-detecting all-reduce, over member buffers in this GPU's HBM.
//
// Member r's bf16 payload sits at bufs[r]; it is ready when flags[r] carries the call's epoch
// (the producer writes the payload, then releases the flag). The sum runs in the member order
// the device array `order` lists ([count, rows...]), in fp32 from 0.0f, rounded once to bf16 by
// torch's rule: core/csrc/slot.cu:118-123,203-223 and core/everserve/reference/arith/ops.py:63-73.
// Floating-point addition is not associative, so the order is part of the result.
//
// Waiting is bounded. Wave 0 of every workgroup reads the flags, one lane per row, with
// system-scope loads (a peer's stores over xGMI, or the host's, land behind this GPU's caches),
// in the same round of loads as the order and the buffer table, and combines the lanes with a
// ballot. While a member is missing it polls again; every 32 polls it reads the wall clock and
// lane 0 reads the ABORT control word. The wait ends when every flag has arrived, when ABORT is
// set, or when the hard timeout passes; a member still missing then contributes zeros, as the
// reference's aborted reads do (slot.cu:148). Workgroups share no word that would end each
// other's waits: each decides for itself, by the flags, ABORT and its own clock. Past the
// BOUND control word (ns, 0 = off) the workgroup writes the rows it still waits for into LATE,
// and the last workgroup that named clears LATE once its wait is over (slot.cu:29-40,174-214).
// Every workgroup is resident at once and bounds its own wait by ABORT and the clock, so they
// give up together, within the skew of their starts.
//
// Early start (EVS_REDUCE_EARLY): a workgroup that finds a member missing at its first read of the
// flags loads the members already in for its first pass before it waits, and after the wait loads
// only the members that came in during it, into the registers that read zeros for them. Every
// load still follows the observation of its member's flag, and the sum still runs in the member
// order, so the result and the outcome equal those of waiting first. After a late flag, the call
// then has only the late members' loads left instead of every member's. Only the kernels of 2 and
// 4 vectors a thread start early: at 1 a workgroup's first pass is too small to gain from it, and
// the unrun path's code slowed the all-in call.
//
// The call's outcome is one word, state[0] = (epoch << 16) | (reason << 8) | late rows, written by
// the last workgroup to count. Each workgroup counts once its wait is over: the outcome is settled
// then, and state[0] is read only after the kernel has completed. The counting runs in a wave of
// its own after the payload's (EVS_REDUCE_CONTROL_WAVE), which moves no payload: a wave's memory
// operations complete in issue order, so in a payload wave each counting atomic held that wave's
// first sum until it returned, and the last of a word's serialised atomics held the call (on
// MI355X the control wave took C5 from 9.34 to 9.02 us a call, 16 Ki elements from 3.16 to 2.98,
// 64 Ki from 3.21 to 2.96, and a grid of one, whose outcome store it also takes, 2.94 to 2.78). How a
// call counts depends on its grid, and is a template parameter chosen at launch, so each kernel
// holds only its own mode's code (on MI355X the code of modes a call does not run cost a small
// grid 0.2-0.3 us, through the registers and schedule of its payload loop):
//   - a grid of one counts nothing: it writes state[0] itself;
//   - a grid of at most EVS_REDUCE_FLAT_MAX workgroups counts in the top word, state[1]: each
//     workgroup ORs its outcome into the high bits and then adds 1 to the low bits, both relaxed
//     atomics on that one location, whose single modification order puts every outcome before
//     the last add; the last adder writes state[0];
//   - a larger grid counts in two levels: workgroup b counts the same way in group word
//     x = b mod 8 (the words 256 bytes apart), and each group's last workgroup carries the
//     group's outcome into the top word. No word then takes more than ceil(workgroups / 8) + 8
//     of the atomics, which on MI355X serialise per address at device scope (one word for every
//     workgroup cost 2.8 us of a 13 us call at 256 workgroups).
// No fence is needed, so no workgroup writes back or invalidates the L2. The counting words return
// to zero in every call, once its last arrival is counted, so the launch needs no memset and a
// captured graph can replay it. These atomics run in one lane; the file is built without the compiler's atomic optimizer,
// whose wave-wide form of them would read each answer at once (with the control wave off, that
// waited out the round trip in front of the payload loads).

#include "common.hpp"

namespace evs {
namespace {

#ifndef EVS_REDUCE_THREADS
#define EVS_REDUCE_THREADS 256
#endif
// bit 0: nontemporal payload loads, bit 1: nontemporal output stores (each byte is touched once)
#ifndef EVS_REDUCE_NT
#define EVS_REDUCE_NT 3
#endif
constexpr int kThreads = EVS_REDUCE_THREADS;  // the threads that move the payload
// 1: each workgroup has one more wave, after the payload's, that does the completion counting. A
// wave's memory operations complete in the order they were issued, so a counting atomic issued by
// a payload wave holds that wave's first sum until the atomic returns, and the atomics of one
// counting word are serialised: the last of a group's arrivals cost the call its wait.
#ifndef EVS_REDUCE_CONTROL_WAVE
#define EVS_REDUCE_CONTROL_WAVE 1
#endif
constexpr bool kControl = EVS_REDUCE_CONTROL_WAVE != 0;
constexpr int kBlockThreads = kThreads + (kControl ? 64 : 0);
constexpr int kMaxRows = EVS_MAX_ROWS;
#ifndef EVS_REDUCE_VPT
#define EVS_REDUCE_VPT 4
#endif
// Every workgroup of the largest grid is resident at once, so that each waits out its own bounded
// wait (a grid past that would time out in turns). The 4-vector kernel's registers leave room for
// two waves a SIMD: two workgroups of 4 waves a CU, one of 5 with the control wave.
#ifndef EVS_REDUCE_MAX_BLOCKS
#define EVS_REDUCE_MAX_BLOCKS (EVS_REDUCE_CONTROL_WAVE ? 256 : 512)
#endif
constexpr int kMaxVpt = EVS_REDUCE_VPT;  // 8-element vectors per thread per pass, at most
constexpr int kMaxBlocks = EVS_REDUCE_MAX_BLOCKS;  // all resident on 256 CUs
constexpr int kCUs = 256;          // MI355X's compute units
constexpr int kPollsPerCheck = 32; // flag polls between clock and ABORT reads
constexpr int kBadOrder = 4;       // reason bit: `order` named a row outside [0, MAX_ROWS)
constexpr int kVectors = 1;        // mode bit: every member buffer 16-byte aligned
constexpr int kEarly = 2;          // mode bit: early start (a member missing at the first read)
constexpr int kDoneBits = 20;      // counting words: workgroups done in bits [0, 20), outcome above
constexpr uint32_t kGroups = 8;    // group counting words
// Grids up to this many workgroups count flat, into the top word: their atomics on one address
// cost less than the second level's round trip. Measured on MI355X, k = 8: at 32 workgroups flat
// ran 3.28 us against 3.54 for two levels; at 64 the two were within the spread between runs;
// at 128 flat ran 4.26 us against 3.48-3.62.
#ifndef EVS_REDUCE_FLAT_MAX
#define EVS_REDUCE_FLAT_MAX 32
#endif
constexpr uint32_t kFlatMax = EVS_REDUCE_FLAT_MAX;
static_assert(kFlatMax >= kGroups && kFlatMax < (1u << 20), "flat counting bound");
// counting modes (a kernel template parameter): a grid of one counts nothing; a grid of at most
// kFlatMax counts in the top word; any grid may count in two levels
constexpr int kCountNone = 0;
constexpr int kCountFlat = 1;
constexpr int kCountTwoLevel = 2;
constexpr int kGroupStride = 32;   // words between counting words (256 bytes)
static_assert(kGroupStride * (1 + kGroups) <= EVS_REDUCE_STATE_WORDS, "state record too small");

// The order of a thread's payload loads: 0 member by member, 1 vector by vector.
#ifndef EVS_REDUCE_LOAD_ORDER
#define EVS_REDUCE_LOAD_ORDER 1
#endif
// How the payload reads are ordered after the flags. 3 (default): every payload load is a buffer
// load at agent scope (sc1), coherent on its own, so no cache is invalidated; issued after the
// flag values returned, it sees what the producer wrote before releasing its flag. 1: one
// acquire fence per workgroup (an L2 invalidate); 2: one per wave; 0: none, right only when every
// payload was written before the launch.
#ifndef EVS_REDUCE_FENCE
#define EVS_REDUCE_FENCE 3
#endif
// Early start (1): a workgroup that finds a member missing at its first read of the flags loads
// its first pass of the members already in, then waits, then loads only the late ones. 0: it
// waits first and loads every member after the wait.
#ifndef EVS_REDUCE_EARLY
#define EVS_REDUCE_EARLY 1
#endif
// Only the kernels of at least this many vectors a thread start early: their first pass is worth
// issuing before the wait. The others wait first, and carry no early-start code.
#ifndef EVS_REDUCE_EARLY_MIN_VPT
#define EVS_REDUCE_EARLY_MIN_VPT 2
#endif
#if EVS_REDUCE_EARLY && EVS_REDUCE_FENCE != 3
#error "early start needs the coherent buffer loads (EVS_REDUCE_FENCE 3)"
#endif
// buffer-load cache policy: sc1 (coherent at agent scope), plus nt when the payload streams
constexpr int kPayloadScope = 16 | ((EVS_REDUCE_NT & 1) ? 2 : 0);
constexpr int kRsrcWord3 = 0x00020000;  // raw buffer resource, dword 3 (gfx9 untyped access)
constexpr int kOutputPolicy = (EVS_REDUCE_NT & 2) ? 2 : 0;  // buffer-store cache policy: nt

typedef uint32_t u32x4 __attribute__((ext_vector_type(4)));

struct ReduceArgs {
  const int64_t* bufs;
  const uint64_t* flags;
  const int32_t* order;
  uint16_t* out;
  int64_t n;
  int64_t nvec;         // 8-element vectors when the vector path is on, else 0
  uint64_t epoch;
  int64_t timeout_ticks;
  int64_t clock_khz;
  uint64_t max_polls;   // a bound on polls that holds even if the clock stood still
  int64_t* ctrl;        // may be null: no abort word, no late word
  uint64_t* state;
};

__device__ __forceinline__ uint64_t load_system(const uint64_t* p) {
  return __hip_atomic_load(p, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_SYSTEM);
}

__device__ __forceinline__ void store_system(int64_t* p, int64_t v) {
  __hip_atomic_store(reinterpret_cast<uint64_t*>(p), static_cast<uint64_t>(v), __ATOMIC_RELAXED,
                     __HIP_MEMORY_SCOPE_SYSTEM);
}

__device__ __forceinline__ float bf16_to_f32(uint32_t bits16) {
  return __uint_as_float(bits16 << 16);
}

// torch's float -> bfloat16: round to nearest even on the bit pattern, any NaN to 0x7FC0.
__device__ __forceinline__ uint32_t f32_to_bf16(float f) {
  const uint32_t u = __float_as_uint(f);
  if ((u & 0x7fffffffu) > 0x7f800000u) return 0x7fc0u;
  return (u + 0x7fffu + ((u >> 16) & 1u)) >> 16;
}

// A buffer resource over `records` bytes from p (uniform across the wave): a raw, untyped view
// whose loads past the end return zeros and whose stores past the end are dropped. The address
// halves go through readfirstlane, which returns a signed int: each is kept as uint32_t before
// the halves are joined, so a low half with bit 31 set does not spill ones into the high half.
__device__ __forceinline__ __amdgpu_buffer_rsrc_t uniform_rsrc(const void* p, int records) {
  const uint64_t a = reinterpret_cast<uint64_t>(p);
  const uint32_t lo = __builtin_amdgcn_readfirstlane(static_cast<uint32_t>(a));
  const uint32_t hi = __builtin_amdgcn_readfirstlane(static_cast<uint32_t>(a >> 32));
  return __builtin_amdgcn_make_buffer_rsrc(
      reinterpret_cast<void*>((static_cast<uint64_t>(hi) << 32) | lo), 0, records, kRsrcWord3);
}

// Count one arrival with `outcome` in the counting word w: OR the outcome into the high bits, then
// add 1 to the low bits. Returns the word as it was before the add.
__device__ __forceinline__ uint64_t arrive(uint64_t* w, uint64_t outcome) {
  if (outcome != 0)
    __hip_atomic_fetch_or(w, outcome << kDoneBits, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
  return __hip_atomic_fetch_add(w, uint64_t{1}, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
}

// Whether the arrival that saw `before` was the last of `arrivals`. The last one gets every
// arrival's outcome in `all` and returns w to zero (the next call touches it only after this
// kernel has ended).
__device__ __forceinline__ bool last(uint64_t* w, uint64_t before, uint32_t arrivals,
                                     uint64_t& all) {
  if ((before & ((uint64_t{1} << kDoneBits) - 1)) != arrivals - 1) return false;
  all = (before >> kDoneBits) & 0xffffu;
  __hip_atomic_store(w, uint64_t{0}, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
  return true;
}

// Wave 0: poll the flags until every wanted member is in (lane q wants the member in order
// position q when `want`; bit q of `missing` is set while it is out), ABORT is set, or the timeout
// passes. Returns the positions still missing. Past BOUND it names the rows still awaited in
// LATE, and the last workgroup that named clears LATE once its wait is over. `reason` gains the
// abort or timeout bit; `late_rows` is the rows still missing when the wait gave up.
__device__ __forceinline__ uint64_t wait_members(const ReduceArgs& a, int lane, bool want,
                                                 int src_lane, int row, uint64_t missing,
                                                 uint32_t& reason, uint32_t& late_rows) {
  bool named = false;
  late_rows = 0;
  const int64_t t0 = wall_clock64();
  for (uint64_t poll = 0;; ++poll) {
    if (poll % kPollsPerCheck == kPollsPerCheck - 1) {
      const int64_t waited = wall_clock64() - t0;
      uint64_t abort = 0, bound_ns = 0;
      if (lane == 0 && a.ctrl != nullptr) {
        abort = load_system(reinterpret_cast<const uint64_t*>(a.ctrl + EVS_ABORT));
        bound_ns = load_system(reinterpret_cast<const uint64_t*>(a.ctrl + EVS_BOUND));
      }
      abort = __shfl(abort, 0);
      bound_ns = __shfl(bound_ns, 0);
      // rows this workgroup still waits for
      uint32_t rows = (missing >> lane) & 1 ? (1u << row) : 0u;
      for (int q = 1; q < kMaxRows; q <<= 1) rows |= __shfl_xor(rows, q);
      late_rows = rows;
      const int64_t waited_ns = waited * 1000000 / a.clock_khz;
      if (a.ctrl != nullptr && static_cast<int64_t>(bound_ns) > 0 &&
          waited_ns > static_cast<int64_t>(bound_ns)) {
        if (lane == 0) {
          if (!named)
            __hip_atomic_fetch_add(a.state + 3, uint64_t{1}, __ATOMIC_RELAXED,
                                   __HIP_MEMORY_SCOPE_AGENT);
          // every check: another workgroup's clear may have raced this one's write
          store_system(a.ctrl + EVS_LATE, static_cast<int64_t>(late_rows));
        }
        named = true;
      }
      if (abort != 0) {
        reason |= EVS_REDUCE_ABORTED;
        break;
      }
      if (waited > a.timeout_ticks || poll >= a.max_polls) {
        reason |= EVS_REDUCE_TIMED_OUT;
        break;
      }
    }
    __builtin_amdgcn_s_sleep(2);
    const uint64_t row_flag = lane < kMaxRows ? load_system(a.flags + lane) : 0;
    const int ready = __shfl(static_cast<int>(row_flag == a.epoch), src_lane);
    missing = __ballot(want && !ready);
    if (missing == 0) break;
  }
  if (missing == 0) late_rows = 0;
  if (named && lane == 0) {
    // the wait is over; the last workgroup that named clears the word
    if (__hip_atomic_fetch_add(a.state + 3, ~uint64_t{0}, __ATOMIC_RELAXED,
                               __HIP_MEMORY_SCOPE_AGENT) == 1)
      store_system(a.ctrl + EVS_LATE, 0);
  }
  return missing;
}

// The bytes a pass's buffer resources span from vector vb: the vectors left, at most 1 GiB.
__device__ __forceinline__ int pass_records(int64_t nvec, int64_t vb) {
  const int64_t left = (nvec - vb) * 16;
  return static_cast<int>(left < (int64_t{1} << 30) ? left : (int64_t{1} << 30));
}

// One pass's payload loads: vector i of every member q, through q's resource (an absent member's
// resource is empty, so its loads return zeros without touching memory).
template <int V>
__device__ __forceinline__ void load_pass(u32x4 (&x)[V][kMaxRows],
                                          const __amdgpu_buffer_rsrc_t (&r)[kMaxRows], int tid) {
  // vector-major (1): vector i's loads from every member come before vector i + 1's, so its sum
  // and store can go out while the later vectors' loads are still in flight
#pragma unroll
  for (int j = 0; j < V * kMaxRows; j++) {
    const int i = EVS_REDUCE_LOAD_ORDER ? j / kMaxRows : j % V;
    const int q = EVS_REDUCE_LOAD_ORDER ? j % kMaxRows : j / V;
    x[i][q] = __builtin_amdgcn_raw_buffer_load_b128(r[q], (i * kThreads + tid) * 16, 0,
                                                    kPayloadScope);
    // keep each vector's loads together, in this order (the scheduler would group them by
    // member otherwise)
    if (EVS_REDUCE_LOAD_ORDER && q == kMaxRows - 1) __builtin_amdgcn_sched_barrier(0);
  }
}

#if EVS_REDUCE_EARLY
// An early start's second round: the vectors of each member q whose bit is set in `late` (the
// same in every lane), loaded over the zeros the first round read for it. Only those members'
// loads are issued, into the registers the first round filled, so the round needs none more.
template <int V>
__device__ __forceinline__ void load_late(u32x4 (&x)[V][kMaxRows],
                                          const uint16_t* const (&late_src)[kMaxRows],
                                          uint32_t late, int64_t vb, int records, int tid) {
#pragma unroll
  for (int q = 0; q < kMaxRows; q++) {
    if ((late >> q) & 1) {
      const __amdgpu_buffer_rsrc_t r = uniform_rsrc(late_src[q] + vb * 8, records);
#pragma unroll
      for (int i = 0; i < V; i++)
        x[i][q] = __builtin_amdgcn_raw_buffer_load_b128(r, (i * kThreads + tid) * 16, 0,
                                                        kPayloadScope);
    }
  }
}
#endif

// Each vector's sum over the members in order, in fp32 from +0.0, rounded to bf16 and stored
// through the output resource `ro`, which ends at the last vector, so a store past it is dropped.
// Adding an absent member's +0.0 changes no sum: the accumulator starts at +0.0 and so is never
// -0.0. Straight-line, so each vector's sum waits only for its own loads.
template <int V>
__device__ __forceinline__ void sum_store(const u32x4 (&x)[V][kMaxRows],
                                          __amdgpu_buffer_rsrc_t ro, int tid) {
#pragma unroll
  for (int i = 0; i < V; i++) {
    float acc[8];
#pragma unroll
    for (int e = 0; e < 8; e++) acc[e] = 0.0f;
#pragma unroll
    for (int q = 0; q < kMaxRows; q++) {
#pragma unroll
      for (int w = 0; w < 4; w++) {
        acc[2 * w] += bf16_to_f32(x[i][q][w] & 0xffffu);
        acc[2 * w + 1] += bf16_to_f32(x[i][q][w] >> 16);
      }
    }
    u32x4 y;
#pragma unroll
    for (int w = 0; w < 4; w++)
      y[w] = f32_to_bf16(acc[2 * w]) | (f32_to_bf16(acc[2 * w + 1]) << 16);
    __builtin_amdgcn_raw_buffer_store_b128(y, ro, (i * kThreads + tid) * 16, 0, kOutputPolicy);
    // the store goes out now, not after the last vector's sum
    if (EVS_REDUCE_LOAD_ORDER) __builtin_amdgcn_sched_barrier(0);
  }
}

// The rest of a call from vector vb on: the passes of the vector path, the elements the vectors
// do not cover, and the completion count (in counting mode C).
template <int V, int C, bool kCounting = !kControl>
__device__ __forceinline__ void finish_call(const ReduceArgs& a,
                                            const uint16_t* const (&src)[kMaxRows], int count,
                                            int64_t nvec, int64_t vb, uint64_t* group_word,
                                            uint64_t group_before, uint32_t group,
                                            uint32_t groups, uint64_t own_outcome) {
  const int tid = threadIdx.x;
  const int64_t stride = static_cast<int64_t>(gridDim.x) * kThreads * V;
  // Two-level counting: the group's last workgroup carries the group's outcome to the top word.
  // It does so right after its first pass's loads are issued: its wait for the group word's
  // answer (counted before the payload) then leaves those loads in flight, and the top word's
  // answer is only read at the end, so no atomic round trip is left for the end of the call.
  constexpr bool two_level = kCounting && C == kCountTwoLevel;
  bool top_sent = false, group_last = false;
  uint64_t group_all = 0, top_before = 0;
  // vectors of 8 elements: one 16-byte load per member
  for (; vb < nvec; vb += stride) {
    const int64_t v0 = vb + tid;
    u32x4 x[V][kMaxRows];
    if (EVS_REDUCE_FENCE == 3) {
      // a buffer resource per member over this pass's vectors: a load past the end returns 0;
      // an absent member (missing, or past the count) gets an empty resource, so no branch
      // separates the loads from their uses
      const int records = pass_records(nvec, vb);
      __amdgpu_buffer_rsrc_t r[kMaxRows];
#pragma unroll
      for (int q = 0; q < kMaxRows; q++)
        r[q] = src[q] != nullptr ? uniform_rsrc(src[q] + vb * 8, records) : uniform_rsrc(a.out, 0);
      load_pass(x, r, tid);
      if (two_level && tid == 0 && !top_sent) {
        // the group word's answer is read here, behind this pass's loads, not before the loop
        asm volatile("" : "+v"(group_before));
        top_sent = true;
        const uint32_t in_group = (gridDim.x - group + groups - 1) / groups;  // b % groups == group
        group_last = last(group_word, group_before, in_group, group_all);
        if (group_last) top_before = arrive(a.state + 1, group_all);
      }
      sum_store(x, uniform_rsrc(a.out + vb * 8, records), tid);
      continue;
    } else {
#pragma unroll
      for (int i = 0; i < V; i++) {
        const int64_t v = v0 + static_cast<int64_t>(i) * kThreads;
#pragma unroll
        for (int q = 0; q < kMaxRows; q++) {
          x[i][q] = u32x4{0u, 0u, 0u, 0u};
          if (v < nvec && src[q] != nullptr)
            x[i][q] = *reinterpret_cast<const u32x4*>(src[q] + v * 8);
        }
      }
    }
#pragma unroll
    for (int i = 0; i < V; i++) {
      const int64_t v = v0 + static_cast<int64_t>(i) * kThreads;
      if (v >= nvec) continue;
      float acc[8];
#pragma unroll
      for (int e = 0; e < 8; e++) acc[e] = 0.0f;
#pragma unroll
      for (int q = 0; q < kMaxRows; q++) {
        if (q >= count) continue;
#pragma unroll
        for (int w = 0; w < 4; w++) {
          acc[2 * w] += bf16_to_f32(x[i][q][w] & 0xffffu);
          acc[2 * w + 1] += bf16_to_f32(x[i][q][w] >> 16);
        }
      }
      u32x4 y;
#pragma unroll
      for (int w = 0; w < 4; w++) y[w] = f32_to_bf16(acc[2 * w]) | (f32_to_bf16(acc[2 * w + 1]) << 16);
      if (EVS_REDUCE_NT & 2)
        __builtin_nontemporal_store(y, reinterpret_cast<u32x4*>(a.out + v * 8));
      else
        *reinterpret_cast<u32x4*>(a.out + v * 8) = y;
    }
  }
  // the elements the vectors do not cover: a tail of fewer than 8, or all of them when a buffer
  // is not 16-byte aligned
  const int64_t first = nvec * 8;
  for (int64_t e = first + static_cast<int64_t>(blockIdx.x) * kThreads + tid; e < a.n;
       e += static_cast<int64_t>(gridDim.x) * kThreads) {
    float acc = 0.0f;
    for (int q = 0; q < count; q++) {
      uint32_t b = 0;
      if (src[q] != nullptr)
        // a global load, not a flat one: member buffers are never LDS
        b = EVS_REDUCE_FENCE == 3
                ? __hip_atomic_load((const __attribute__((address_space(1))) uint16_t*)(src[q] + e),
                                    __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT)
                : src[q][e];
      acc += bf16_to_f32(b);
    }
    a.out[e] = static_cast<uint16_t>(f32_to_bf16(acc));
  }

  if (kCounting && tid == 0) {
    uint64_t outcome = own_outcome;
    bool all_in = true;  // this workgroup has every workgroup's outcome in `outcome`
    if (two_level) {
      if (!top_sent) {  // no vector pass ran here: carry the group's outcome now
        const uint32_t in_group = (gridDim.x - group + groups - 1) / groups;
        group_last = last(group_word, group_before, in_group, group_all);
        if (group_last) top_before = arrive(a.state + 1, group_all);
      }
      all_in = group_last && last(a.state + 1, top_before, groups, outcome);
    } else if (C == kCountFlat) {
      all_in = last(group_word, group_before, gridDim.x, outcome);  // group_word is the top word
    }
    if (all_in)
      __hip_atomic_store(a.state + 0, (a.epoch << 16) | outcome, __ATOMIC_RELAXED,
                         __HIP_MEMORY_SCOPE_SYSTEM);
  }
}

// The control wave's counting, in its lane 0: this workgroup's arrival with outcome `own`, as
// finish_call counts it in the payload's first wave, and for the call's last arrival the outcome
// word. Its wave issues nothing else, so each atomic's answer waits behind no payload load, and
// the chain ends long before the payload does.
template <int C>
__device__ __forceinline__ void count_arrival(const ReduceArgs& a, uint64_t* group_word,
                                              uint32_t group, uint32_t groups, uint64_t own) {
  uint64_t outcome = own;
  bool all_in = true;  // this arrival has every workgroup's outcome in `outcome`
  if (C == kCountTwoLevel) {
    const uint64_t before = arrive(group_word, own);
    const uint32_t in_group = (gridDim.x - group + groups - 1) / groups;  // b % groups == group
    uint64_t group_all = 0;
    all_in = last(group_word, before, in_group, group_all);
    if (all_in) all_in = last(a.state + 1, arrive(a.state + 1, group_all), groups, outcome);
  } else if (C == kCountFlat) {
    all_in = last(group_word, arrive(group_word, own), gridDim.x, outcome);  // the top word
  }
  if (all_in)
    __hip_atomic_store(a.state + 0, (a.epoch << 16) | outcome, __ATOMIC_RELAXED,
                       __HIP_MEMORY_SCOPE_SYSTEM);
}

template <int V, int C>
__global__ __launch_bounds__(kBlockThreads) void local_reduce(ReduceArgs a) {
  constexpr bool kStartsEarly = EVS_REDUCE_EARLY && V >= EVS_REDUCE_EARLY_MIN_VPT;
  __shared__ const uint16_t* s_src[kMaxRows];  // member in order position q, or null: missing
  __shared__ int s_count;
  __shared__ int s_mode;                         // kVectors | kEarly
  __shared__ uint32_t s_outcome;                 // reason << 8 | late rows

  const int tid = threadIdx.x;
  const int64_t first_vb = static_cast<int64_t>(blockIdx.x) * kThreads * V;  // first vector
  // wave 0's view of the members (lane q: order position q), kept for an early start's wait
  int row = -1, src_lane = 0;
  bool valid = false;
  int64_t addr = 0;
  uint64_t missing = 0;
  uint32_t reason = 0;
  if (tid < 64) {
    const int lane = tid;
    // One round of independent loads: the order words, the buffer table and every row's flag
    // (lane r holds row r's), so a call whose members are all in costs one memory latency here.
    const int o = lane <= kMaxRows ? a.order[lane] : 0;
    const int64_t row_addr = lane < kMaxRows ? a.bufs[lane] : 0;
    const uint64_t row_flag = lane < kMaxRows ? load_system(a.flags + lane) : 0;
    int count = __shfl(o, 0);
    count = count < 0 ? 0 : (count > kMaxRows ? kMaxRows : count);
    // lane q < count stands for the member in order position q
    const int listed_row = __shfl(o, (1 + lane) & 63);
    const bool listed = lane < count;
    row = listed ? listed_row : -1;
    valid = listed && row >= 0 && row < kMaxRows;
    reason = __ballot(listed && !valid) ? kBadOrder : 0;
    src_lane = valid ? row : 0;

    // every lane takes part in every shuffle: a lane left out supplies no value to read
    const int ready = __shfl(static_cast<int>(row_flag == a.epoch), src_lane);
    missing = __ballot(valid && !ready);
    const int64_t mapped_addr = __shfl(row_addr, src_lane);
    addr = valid ? mapped_addr : 0;
    const bool unaligned = __ballot((addr & 15) != 0) != 0;
    // Early start: with a member missing, every wave loads this workgroup's first pass of the
    // members already in, and this wave waits for the rest after issuing its share.
    const bool early = kStartsEarly && missing != 0 && !unaligned && first_vb < a.nvec;
    uint32_t late_rows = 0;
    if (missing != 0 && !early)
      missing = wait_members(a, lane, valid, src_lane, row, missing, reason, late_rows);
    if (lane < kMaxRows) {
      const bool have = valid && !((missing >> lane) & 1);
      s_src[lane] = have ? reinterpret_cast<const uint16_t*>(addr) : nullptr;
    }
    if (lane == 0) {
      s_count = count;
      s_mode = (unaligned ? 0 : kVectors) | (early ? kEarly : 0);
      s_outcome = (reason << 8) | late_rows;
    }
    // the flags were read with relaxed loads: order the payload reads after them
    if (EVS_REDUCE_FENCE == 1) __builtin_amdgcn_fence(__ATOMIC_ACQUIRE, "agent");
  }
  __syncthreads();
  if (EVS_REDUCE_FENCE == 2) __builtin_amdgcn_fence(__ATOMIC_ACQUIRE, "agent");
  // This workgroup's outcome is settled once its wait is over, so it is counted then: the
  // counting atomic's round trip then overlaps the payload instead of following it. state[0] is
  // read only once the kernel has completed, when every workgroup's payload is written too.
  // Flat counting puts every workgroup in the top word; a grid of one counts nothing (its outcome
  // is the call's).
  const uint32_t groups = gridDim.x < kGroups ? gridDim.x : kGroups;
  const uint32_t group = blockIdx.x % groups;
  uint64_t* const group_word =
      C == kCountTwoLevel ? a.state + kGroupStride * (1 + group) : a.state + 1;
  constexpr bool counts = C != kCountNone;
  uint64_t group_before = 0;
  const int mode = s_mode;
  const bool waiting = kStartsEarly && (mode & kEarly) != 0;
  if constexpr (kControl) {
    if (tid >= kThreads) {  // the control wave: it counts, and moves no payload
      if (waiting) __syncthreads();  // the early start's barrier, after wave 0's wait
      if (tid == kThreads) count_arrival<C>(a, group_word, group, groups, s_outcome);
      return;
    }
  }
  if (!kControl && tid == 0 && !waiting && counts) group_before = arrive(group_word, s_outcome);

  const int count = s_count;
  const int64_t nvec = (mode & kVectors) ? a.nvec : 0;
  int64_t vb = first_vb;
  const uint16_t* src[kMaxRows];
#pragma unroll
  for (int q = 0; q < kMaxRows; q++) src[q] = q < count ? s_src[q] : nullptr;
#if EVS_REDUCE_EARLY
  if constexpr (kStartsEarly) {
    __shared__ const uint16_t* s_late[kMaxRows];  // member q if it came in during the wait
    __shared__ uint32_t s_came;                     // the order positions s_late names
    // unlikely: the call whose members are all in at the first read does not run this
    if (__builtin_expect(waiting, 0)) {
      // The first pass in two rounds of loads: the members that were in at the first read, issued
      // now, and after the wait the members that came in during it. A member that never came in
      // reads as zeros in both. The wait ends on the same events as the one above, so the outcome
      // and the sum equal a wait-then-load call's.
      u32x4 x[V][kMaxRows];
      const int records = pass_records(nvec, vb);
      __amdgpu_buffer_rsrc_t r[kMaxRows];
#pragma unroll
      for (int q = 0; q < kMaxRows; q++)
        r[q] = src[q] != nullptr ? uniform_rsrc(src[q] + vb * 8, records) : uniform_rsrc(a.out, 0);
      load_pass(x, r, tid);
      if (tid < 64) {
        const int lane = tid;
        uint32_t late_rows = 0;
        const uint64_t still = wait_members(a, lane, valid && ((missing >> lane) & 1), src_lane,
                                            row, missing, reason, late_rows);
        const uint64_t came = missing & ~still;  // positions that came in during the wait
        if (lane < kMaxRows)
          s_late[lane] = (came >> lane) & 1 ? reinterpret_cast<const uint16_t*>(addr) : nullptr;
        if (lane == 0) {
          s_came = static_cast<uint32_t>(came);
          s_outcome = (reason << 8) | late_rows;
        }
      }
      __syncthreads();
      if (!kControl && tid == 0 && counts) group_before = arrive(group_word, s_outcome);
      load_late(x, s_late, __builtin_amdgcn_readfirstlane(s_came), vb, records, tid);
      sum_store(x, uniform_rsrc(a.out + vb * 8, records), tid);
      vb += static_cast<int64_t>(gridDim.x) * kThreads * V;
      // the later passes and the element tail read every member that is in; this path ends here,
      // so the common path's code stays as it is
#pragma unroll
      for (int q = 0; q < kMaxRows; q++)
        if (src[q] == nullptr) src[q] = s_late[q];
      finish_call<V, C>(a, src, count, nvec, vb, group_word, group_before, group, groups,
                        s_outcome);
      return;
    }
  }
#endif

  finish_call<V, C>(a, src, count, nvec, vb, group_word, group_before, group, groups, s_outcome);
}

int64_t g_clock_khz[64];

int clock_khz(int64_t* khz) {
  int dev = 0;
  EVS_HIP(hipGetDevice(&dev));
  EVS_REQUIRE(dev >= 0 && dev < 64, "device %d out of range", dev);
  if (g_clock_khz[dev] == 0) {
    int rate = 0;
    EVS_HIP(hipDeviceGetAttribute(&rate, hipDeviceAttributeWallClockRate, dev));
    EVS_REQUIRE(rate > 0, "device %d reports no wall clock rate", dev);
    g_clock_khz[dev] = rate;
  }
  *khz = g_clock_khz[dev];
  return EVS_OK;
}

}  // namespace

int wall_clock_khz(int64_t* khz) { return clock_khz(khz); }

}  // namespace evs

extern "C" int evs_local_reduce(const int64_t* bufs, const uint64_t* flags, const int32_t* order,
                                void* out, int64_t n, uint64_t epoch, int64_t timeout_ns,
                                int64_t* ctrl, uint64_t* state, void* stream) {
  evs::clear_error();
  EVS_REQUIRE(bufs != nullptr && flags != nullptr && order != nullptr && state != nullptr,
              "evs_local_reduce: null pointer");
  EVS_REQUIRE(n >= 0, "evs_local_reduce: negative element count");
  EVS_REQUIRE(n == 0 || out != nullptr, "evs_local_reduce: null output");
  EVS_REQUIRE((reinterpret_cast<int64_t>(out) & 1) == 0, "evs_local_reduce: unaligned output");
  int64_t khz = 0;
  int rc = evs::clock_khz(&khz);
  if (rc != EVS_OK) return rc;
  if (timeout_ns <= 0) timeout_ns = 1000000000;
  EVS_REQUIRE(timeout_ns < (int64_t{1} << 50), "evs_local_reduce: timeout too large");
  evs::ReduceArgs a{};
  a.bufs = bufs;
  a.flags = flags;
  a.order = order;
  a.out = static_cast<uint16_t*>(out);
  a.n = n;
  // the member buffers live in a device table the host does not read: the kernel checks their
  // alignment itself and takes the element path when one is not 16-byte aligned
  a.nvec = evs::aligned16(reinterpret_cast<int64_t>(out)) ? n / 8 : 0;
  a.epoch = epoch;
  a.timeout_ticks = timeout_ns / 1000 * khz / 1000;
  a.clock_khz = khz;
  a.max_polls = static_cast<uint64_t>(timeout_ns / 50) + 4096;
  a.ctrl = ctrl;
  a.state = state;
  // Vectors per thread: the fewest (1, 2, then kMaxVpt) that keep the grid within one workgroup
  // a CU. A thread's loads of one vector from every member go out together; more vectors a
  // thread than the data needs only add loads that read nothing, and fewer, fatter workgroups
  // than CUs leave CUs idle (measured on MI355X: 1 vector a thread is fastest up to 512 Ki
  // elements, 2 at 1 Mi, 4 at 2 Mi).
  int vpt = evs::kMaxVpt;
  for (const int v : {1, 2}) {
    if (v < vpt && (a.nvec + int64_t{evs::kThreads} * v - 1) / (int64_t{evs::kThreads} * v) <=
                       evs::kCUs) {
      vpt = v;
      break;
    }
  }
  const int64_t per_block = static_cast<int64_t>(evs::kThreads) * vpt;
  int64_t blocks = (a.nvec + per_block - 1) / per_block;
  const int64_t tail_blocks = (n - a.nvec * 8 + evs::kThreads - 1) / evs::kThreads;
  if (tail_blocks > blocks) blocks = tail_blocks;
  if (blocks < 1) blocks = 1;
  if (blocks > evs::kMaxBlocks) blocks = evs::kMaxBlocks;
  const dim3 grid(static_cast<uint32_t>(blocks)), block(evs::kBlockThreads);
  hipStream_t s = evs::as_stream(stream);
  // The counting mode follows the grid. Two-level counting is right for any grid, so the wider
  // kernels, whose grids are past the flat bound whenever the rule above picks them, carry only it.
  if (vpt == 1 && blocks == 1)
    hipLaunchKernelGGL((evs::local_reduce<1, evs::kCountNone>), grid, block, 0, s, a);
  else if (vpt == 1 && blocks <= evs::kFlatMax)
    hipLaunchKernelGGL((evs::local_reduce<1, evs::kCountFlat>), grid, block, 0, s, a);
  else if (vpt == 1)
    hipLaunchKernelGGL((evs::local_reduce<1, evs::kCountTwoLevel>), grid, block, 0, s, a);
  else if (vpt == 2)
    hipLaunchKernelGGL((evs::local_reduce<2, evs::kCountTwoLevel>), grid, block, 0, s, a);
  else
    hipLaunchKernelGGL((evs::local_reduce<evs::kMaxVpt, evs::kCountTwoLevel>), grid, block, 0, s,
                       a);
  EVS_LAUNCHED("evs_local_reduce");
  return EVS_OK;
}
