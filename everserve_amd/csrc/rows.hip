// The step's KV rows between the paged cache and a staging buffer, on gfx950.
//
// Gather (the snapshot) reads each (layer, head slot, slot) K and V half-row out of a paged cache
// and writes it into a buffer laid out [layers, heads, capacity, 2, head_dim]; scatter (the
// restore) is its inverse. A cache layout is five strides (block, offset in block, head slot,
// K-or-V, element), so the three paged layouts and strided views share one kernel
// (core/everserve/state/kvcopy.py:105-116; the reference kernels are core/csrc/gather.cu:29-71).
//
// Work is cut into small tiles of (one layer, HG consecutive held heads, TS consecutive slots).
// One workgroup owns a tile: its first TS threads turn the tile's slot ids (or block ids) into
// byte offsets inside a layer, the first HG threads the head slots, both into LDS, so each moved
// word costs two LDS reads and no 64-bit division. Each thread then moves VPT words at a time,
// every load in flight before the first store. A word is 16 bytes when every half-row is
// contiguous and 16-byte aligned on both sides (bf16 d=128: 16 words a half-row, fp8 d=128: 8),
// else one element. Within a tile the words run along the staging buffer (K then V of one row,
// row after row), so a wave stores whole rows: 1 KiB contiguous for bf16 d=128. For the gather
// the tile numbers run through a slot range's head groups first, so the workgroups reading the
// heads of one cache block (adjacent in every paged layout) are neighbours, dealt round-robin to
// the XCDs; the slot and pair scatters' XCD remap (xcd_tile) keeps runs of 64 neighbouring tiles
// on one XCD, and the range scatter's gives each XCD one contiguous part of the grid. Tiles are
// kept small (a few KiB) and numerous: on MI355X many short independent workgroups keep more
// bytes in flight than fewer long ones. Measured and rejected:
// a persistent grid with prefetched indices, and an LDS-staged transpose that reads a tile in
// cache order and writes it in staging order (both slower on every config); for the scatter,
// words in cache order and issuing a tile's loads before its slot ids are read (both slower);
// fewer workgroups per CU (unused LDS as a cap), which speeds a plain copy up by 8 % at 8 KiB per
// workgroup but slows these kernels, whose index prologue needs every resident workgroup to hide
// its latency; each wave reading its own rows' ids with scalar loads, no LDS and no barrier
// (2 % slower: the per-lane choice among the wave's rows costs more than the barrier).

#include "common.hpp"

namespace evs {
namespace {

// Tuning, chosen by measurement on MI355X (the defaults); the macros let a sweep build variants
// side by side.
#ifndef EVS_GATHER_THREADS
#define EVS_GATHER_THREADS 256
#endif
#ifndef EVS_SCATTER_THREADS
#define EVS_SCATTER_THREADS 128
#endif
// Words per thread per pass, per direction: all of a pass's loads are issued before its stores.
#ifndef EVS_GATHER_VPT
#define EVS_GATHER_VPT 2
#endif
#ifndef EVS_SCATTER_VPT
#define EVS_SCATTER_VPT 2
#endif
// Per direction, bit 0: nontemporal loads, bit 1: nontemporal stores. Every byte here is touched
// once, so no line is worth keeping in L2 or the Infinity Cache. For the scatter in staged order
// the nontemporal row loads also keep the slot ids in L2: each of a slot range's 8 head tiles
// reads them, far apart in time, and with plain row loads streaming through L2 every read missed
// (HBM traffic 1.0078x the algorithmic bytes at C4; 1.00002x with the loads nontemporal, and
// 5,646-5,657 against 5,627-5,653 GB/s, interleaved rounds on one box). The range scatter reads
// no ids, and its nontemporal loads ran at 5,900 against 5,852 GB/s (C4, one box).
#ifndef EVS_GATHER_NT
#define EVS_GATHER_NT 3
#endif
#ifndef EVS_SCATTER_NT
#define EVS_SCATTER_NT 3
#endif
#ifndef EVS_RANGES_NT
#define EVS_RANGES_NT EVS_SCATTER_NT
#endif
// The gather's 16-byte stores also carry sc1, device scope: written through this XCD's L2, which
// then holds no dirty lines of the staging buffer to write back later. Measured on MI355X (9
// interleaved rounds, the bytes equal): C2 6,087 against 6,003 GB/s on random blocks and 6,168
// against 6,084 on sorted ones, C3 6,147 against 6,045. The scatter's stores were unchanged by it
// (5,619 either way), and keep the plain nontemporal bit. 0: the plain bit for the gather too.
#ifndef EVS_GATHER_STORE_SC1
#define EVS_GATHER_STORE_SC1 1
#endif
// Word order in a tile, per direction. 0: along the cache in the common layouts (a wave covers
// consecutive heads of one slot, K then V); 1: along the staging buffer (whole staged rows).
#ifndef EVS_GATHER_ORDER
#define EVS_GATHER_ORDER 1
#endif
#ifndef EVS_SCATTER_ORDER
#define EVS_SCATTER_ORDER 1
#endif
// Workgroups are dealt to the XCDs round-robin by id, so consecutive tiles (the tiles of one cache
// block) would each run on another XCD. The chunk per direction remaps tile numbers: 0 leaves
// them; G > 0 gives each XCD G consecutive tiles of every run of kXcds * G; -1 gives each XCD one
// contiguous range of the whole grid.
// The gather leaves the round-robin dealing: against runs of 64 it measured 1.3 % faster on C2's
// random blocks, 3.1 % on sorted ones, 1.2-1.7 % on C3 and 4 % at decode size (5 interleaved
// rounds, three boxes).
#ifndef EVS_GATHER_XCD_CHUNK
#define EVS_GATHER_XCD_CHUNK 0
#endif
// A gather whose tiles cover every held head (one head group, as on a rank holding one KV head)
// numbers its tiles along the slots alone, and there runs of 16 tiles per XCD (128 KiB of staged
// rows each) beat round-robin. 7 interleaved rounds on each of two boxes: one bf16 head, 80
// layers, 65,536 slots 6,184 / 6,218 against 5,946 / 5,978 GB/s (runs of 4 / 8 on the first:
// 5,771 / 5,902); C3's fp8 head 6,138 / 6,216 against 6,030 / 6,131. With several head groups
// the round-robin default stays (C2 6,078 against 6,074 under this switch's build).
#ifndef EVS_GATHER_XCD_CHUNK_ONE_GROUP
#define EVS_GATHER_XCD_CHUNK_ONE_GROUP 16
#endif
#ifndef EVS_SCATTER_XCD_CHUNK
#define EVS_SCATTER_XCD_CHUNK 64
#endif
// The scatter of written ranges (staged rows to the slots of (start, count) ranges, which ascend
// in a restore) gives each XCD one contiguous part of the grid, so that the XCDs write the cache
// in 8 streams that each run front to back. On ascending slots that measured faster than runs of
// 64 on every box tried: a restore's chunk (1 layer, 8 heads, 65,536 slots) 6,339 against 5,735
// GB/s for an isolated launch; 16 layers of C4's cache 5,801-6,144 against 5,447-5,537. For the
// slot scatter's permuted slots it depended on the box (16 layers: 4.8 % faster on two runs, 2.4 %
// slower on another; C4's 32 layers 2 % slower), so that one keeps runs of 64.
#ifndef EVS_RANGES_XCD_CHUNK
#define EVS_RANGES_XCD_CHUNK -1
#endif
constexpr uint32_t kXcds = 8;
// The pair scatter (a staged row per listed slot, listed in the order the caller wants written):
// its tiles span all heads (2 slots x 8 heads at bf16 d=128, 8 KiB) and its words run along the
// cache, so that a caller listing its slots in increasing order writes each layer's cache front
// to back. A tile is one pass (256 threads x 2 words) and its reads, which are random, are
// nontemporal, as the gather's are. On C4's permuted block table with the pairs in slot order it
// measured 5,994 GB/s, against 5,660 for the scatter in staged order on the same box.
#ifndef EVS_PAIRS_TILE_WORDS
#define EVS_PAIRS_TILE_WORDS 512
#endif
#ifndef EVS_PAIRS_HEADS_PER_TILE
#define EVS_PAIRS_HEADS_PER_TILE 0
#endif
#ifndef EVS_PAIRS_ORDER
#define EVS_PAIRS_ORDER 0
#endif
#ifndef EVS_PAIRS_XCD_CHUNK
#define EVS_PAIRS_XCD_CHUNK 64
#endif
#ifndef EVS_PAIRS_THREADS
#define EVS_PAIRS_THREADS 256
#endif
#ifndef EVS_PAIRS_NT
#define EVS_PAIRS_NT 3  // its reads are random, as the gather's are: nontemporal both ways
#endif
#ifndef EVS_PAIRS_VPT
#define EVS_PAIRS_VPT 2
#endif
// Tile shape per direction: words a tile aims at, heads it covers (0: all), head groups fastest.
#ifndef EVS_GATHER_TILE_WORDS
#define EVS_GATHER_TILE_WORDS 512
#endif
#ifndef EVS_GATHER_HEADS_PER_TILE
#define EVS_GATHER_HEADS_PER_TILE 2
#endif
#ifndef EVS_GATHER_GROUP_FASTEST
#define EVS_GATHER_GROUP_FASTEST 1
#endif
#ifndef EVS_SCATTER_TILE_WORDS
#define EVS_SCATTER_TILE_WORDS 256
#endif
#ifndef EVS_SCATTER_HEADS_PER_TILE
#define EVS_SCATTER_HEADS_PER_TILE 1
#endif
#ifndef EVS_SCATTER_GROUP_FASTEST
#define EVS_SCATTER_GROUP_FASTEST 0
#endif
#ifndef EVS_RANGES_GROUP_FASTEST
#define EVS_RANGES_GROUP_FASTEST EVS_SCATTER_GROUP_FASTEST
#endif

constexpr int kMaxTileSlots = 64;
constexpr int kMaxHeads = 256;      // LDS table of head offsets

enum Dir : int { kGather = 0, kScatter = 1 };
// kBySlots: row t of a layer's staging goes to (or comes from) slot slots[t]; kByBlocks: row t is
// offset t % bs of the (t / bs)-th listed block; kByPairs (scatter): staged row rows_of[i] goes
// to slot slots[i]; kByRanges (scatter): row t goes to slot starts[k] + t - first_rows[k] of the
// range k with first_rows[k] <= t < first_rows[k + 1].
enum Index : int { kBySlots = 0, kByBlocks = 1, kByPairs = 2, kByRanges = 3 };

constexpr int threads_of(int d, int i) {
  return i == kByPairs ? EVS_PAIRS_THREADS : d == kGather ? EVS_GATHER_THREADS : EVS_SCATTER_THREADS;
}
constexpr int vpt_of(int d, int i) {
  return i == kByPairs ? EVS_PAIRS_VPT : d == kGather ? EVS_GATHER_VPT : EVS_SCATTER_VPT;
}
constexpr int nt_of(int d, int i) {
  return i == kByPairs    ? EVS_PAIRS_NT
         : i == kByRanges  ? EVS_RANGES_NT
         : d == kGather    ? EVS_GATHER_NT
                           : EVS_SCATTER_NT;
}
constexpr int order_of(int d) { return d == kGather ? EVS_GATHER_ORDER : EVS_SCATTER_ORDER; }
constexpr int word_order(int d, int i) { return i == kByPairs ? EVS_PAIRS_ORDER : order_of(d); }
static_assert(threads_of(kGather, kBySlots) >= kMaxTileSlots &&
                  threads_of(kScatter, kBySlots) >= kMaxTileSlots &&
                  threads_of(kScatter, kByPairs) >= kMaxTileSlots,
              "the first TS threads fill a tile's slot offsets: a workgroup needs kMaxTileSlots");

typedef uint32_t u32x4 __attribute__((ext_vector_type(4)));

// one cell per word of a pass, at the widest pass
constexpr int kSinkWords = 1024;
static_assert(threads_of(kGather, kBySlots) * vpt_of(kGather, kBySlots) <= kSinkWords &&
                  threads_of(kScatter, kBySlots) * vpt_of(kScatter, kBySlots) <= kSinkWords &&
                  threads_of(kScatter, kByPairs) * vpt_of(kScatter, kByPairs) <= kSinkWords,
              "the sink holds one cell per word of a pass");

// Where a gathered word that moves nothing goes: a lane with no word (a slot past n, a word past
// the tile) loads from and stores into its own 16-byte cell here instead of branching around the
// access. With no branch between them, a thread's loads are all issued before its first store and
// each store waits only for its own data; a branch around each access makes the compiler wait for
// every memory operation in flight before each store, which serialises a thread's stores (the
// gather measured 1 % faster without). The scatter keeps the branches: its scattered stores ran
// 0.5-1.5 % faster serialised than all in flight. The contents are never read as data.
// Workgroups take one of kSinkCopies regions by id: with one region shared by all, a call whose
// tiles leave most lanes idle (a decode step of 1-4 slots) sent every such store to the same
// 16 KiB, and so to the same few memory channels, and took 4.5 us where 8 slots took 2.45.
constexpr int kSinkCopies = 64;
__device__ u32x4 g_sink[kSinkCopies * kSinkWords];

struct RowsArgs {
  const int64_t* layer_ptrs;  // device: each layer's cache base address
  const int64_t* slots;       // kBySlots: device slot ids
  const int32_t* blocks;      // kByBlocks: device block ids
  const int64_t* heads;       // device head slots
  char* rows;                 // the staging buffer, [L, H, cap, 2, d]
  int64_t* slots_out;         // kByBlocks: the expanded slot ids, or null
  const int64_t* rows_of;     // kByPairs: the staged row of each listed slot
  const int64_t* starts;      // kByRanges: device, each range's first slot
  const int64_t* first_rows;  // kByRanges: device, each range's first row, then n
  int64_t nranges;            // kByRanges
  int64_t n;                  // slots moved per layer
  int64_t cap;                // staging capacity (rows per (layer, head))
  int64_t half_bytes;         // d * elem
  int64_t sb, so, sh, skv;    // cache strides in bytes: block, offset, head, K-or-V
  int64_t sj;                 // cache bytes between consecutive words of a half-row
  int64_t bs;                 // slots per block
  int bs_shift;               // log2(bs) when bs is a power of two, else -1
  int H;
  int HG;                     // heads per tile (a tile's heads are HG consecutive of `heads`)
  int TS;                     // slots per tile
  int group_fastest;          // tile numbers run through head groups first
  int xcd_chunk;              // tiles per XCD per run (see xcd_tile)
  uint32_t tile_words;        // TS * HG * 2 * W
  FastDiv div_w;              // words per half-row
  FastDiv div_h;              // heads per tile
  FastDiv div_ts;             // slots per tile
  FastDiv div_tiles;          // slot tiles per (layer, head group)
  FastDiv div_groups;         // head groups
};

// Every address these kernels touch is global memory (device, or host memory mapped for the
// device), but the cache's come out of a table of integers, so the compiler would emit flat
// accesses; the casts to address space 1 make them global ones.
template <typename T>
using global_ptr = __attribute__((address_space(1))) T*;

template <typename T, bool kNt>
__device__ __forceinline__ T load_word(const char* p) {
  const global_ptr<const T> g = (global_ptr<const T>)(p);
  if (kNt) return __builtin_nontemporal_load(g);
  return *g;
}

template <typename T, bool kNt, bool kSc1 = false>
__device__ __forceinline__ void store_word(char* p, T v) {
  const global_ptr<T> g = (global_ptr<T>)(p);
  if constexpr (kNt && kSc1 && sizeof(T) == 16)
    // No builtin sets the scope bits on a plain store; the word and the address are the asm's
    // inputs, so the compiler waits for the loaded word before it, as for any store. A store of
    // more than 64 bits reads its data registers after it issues, so a VALU write to them needs
    // one wait state after it; the compiler's hazard check does not see inside the asm, so the
    // s_nop gives that wait state whatever is scheduled next.
    asm volatile("global_store_dwordx4 %0, %1, off sc1 nt\n\ts_nop 0" : : "v"(g), "v"(v)
                 : "memory");
  else if (kNt)
    __builtin_nontemporal_store(v, g);
  else
    *g = v;
}

__device__ __forceinline__ int64_t block_of(int64_t s, const RowsArgs& a) {
  return a.bs_shift >= 0 ? (s >> a.bs_shift) : s / a.bs;
}

__device__ __forceinline__ int64_t offset_in_block(int64_t s, const RowsArgs& a) {
  return a.bs_shift >= 0 ? (s & (a.bs - 1)) : s % a.bs;
}

// Which (layer, head group, slot tile) a tile number names.
struct TileId {
  uint32_t layer, group, tile;
};

// The tile workgroup id b runs, ids being dealt to kXcds XCDs round-robin (x = b % kXcds).
//   chunk > 0: in each run of kXcds * chunk ids, XCD x takes tiles [x chunk, (x + 1) chunk) of the
//              run; a last partial run keeps its ids;
//   chunk < 0: XCD x takes the contiguous tiles [x (q + 1), ...) when x < r, after them q each,
//              for grid = kXcds q + r.
// Both are bijections of [0, grid).
__device__ __forceinline__ uint32_t xcd_tile(uint32_t b, uint32_t grid, int chunk) {
  if (chunk == 0) return b;
  const uint32_t x = b % kXcds, local = b / kXcds;
  if (chunk > 0) {
    const uint32_t run = kXcds * static_cast<uint32_t>(chunk);
    if (b >= grid / run * run) return b;
    const uint32_t g = static_cast<uint32_t>(chunk);
    return (b / run) * run + x * g + local % g;
  }
  const uint32_t q = grid / kXcds, r = grid % kXcds;
  return x < r ? x * (q + 1) + local : r * (q + 1) + (x - r) * q + local;
}

__device__ __forceinline__ TileId tile_id(const RowsArgs& a, uint32_t b) {
  TileId id;
  uint32_t q;
  if (a.group_fastest) {
    // head groups fastest: the tiles that read one slot range's heads run side by side
    a.div_groups.divmod(b, q, id.group);
    a.div_tiles.divmod(q, id.layer, id.tile);
  } else {
    a.div_tiles.divmod(b, q, id.tile);
    a.div_groups.divmod(q, id.layer, id.group);
  }
  return id;
}

// The slot of staged row t (0 <= t < n) in the written ranges: the last range k whose first row
// is at most t (first_rows ascending, first_rows[0] = 0, the last entry n), so an empty range is
// passed over. Ranges that break these rules give slots the caller did not mean, as wrong slot ids
// would; a negative one moves nothing. Found for a tile's rows by the tile's first wave together:
// every lane of wave 0 calls it, lane i with row t = t0 + i (rows past the tile's repeat its last;
// t0 <= t < n). The range
// of t0 is found by a 64-way search, each level one read a lane and a ballot (two levels up to
// 4,096 ranges, where bisection takes a dependent read for each of 12 halvings); then the 64
// ranges from there are read at once, first rows and starts, and each lane picks its own among
// them with shuffles. A lane whose row lies past those 64 ranges (only when many ranges are
// empty) bisects the rest. Every read stays inside first_rows[0 .. nranges] and
// starts[0 .. nranges - 1] whatever the arrays hold.
__device__ __forceinline__ int64_t wave_slot_in_ranges(const RowsArgs& a, int64_t t0, int64_t t) {
  const int64_t nr = a.nranges;
  if (nr == 1) return a.starts[0] + (t - a.first_rows[0]);
  const int lane = static_cast<int>(threadIdx.x & 63);
  int64_t lo = 0, hi = nr;  // the range of t0 is in [lo, hi)
  while (hi - lo > 1) {
    const int64_t step = (hi - lo + 63) >> 6;
    const int64_t p = lo + lane * step;
    const uint64_t le = __ballot(p < hi && a.first_rows[p] <= t0);
    lo += le != 0 ? static_cast<int64_t>(63 - __builtin_clzll(le)) * step : 0;
    hi = lo + step < hi ? lo + step : hi;
  }
  const int64_t k = lo + lane;
  const int64_t fr = a.first_rows[k < nr ? k : nr];  // first_rows[nr] = n: past every row
  const int64_t st = a.starts[k < nr ? k : nr - 1];
  // c: the last of the 64 whose first row is at most t
  int c = 0;
  for (int b = 32; b >= 1; b >>= 1) {
    const int64_t v = __shfl(fr, c + b);
    if (v <= t) c += b;
  }
  int64_t slot = __shfl(st, c) + (t - __shfl(fr, c));
  if (c == 63 && lo + 63 < nr - 1) {
    int64_t l2 = lo + 63, h2 = nr;
    while (h2 - l2 > 1) {
      const int64_t mid = (l2 + h2) >> 1;
      if (a.first_rows[mid] <= t)
        l2 = mid;
      else
        h2 = mid;
    }
    slot = a.starts[l2] + (t - a.first_rows[l2]);
  }
  return slot;
}

// The index entry row t of a layer needs: its slot id, or in the block-table path its block's id.
// It is read at a clamped position (n >= 1 here), so that the read needs no branch; the caller
// discards what it read for a row past n.
template <int I>
__device__ __forceinline__ int64_t index_entry(const RowsArgs& a, int64_t t) {
  const int64_t tc = t < a.n ? t : a.n - 1;
  if (I == kByBlocks) return a.blocks[block_of(tc, a)];
  return a.slots[tc];
}

// Byte offset of slot t's row inside a layer, or -1 when nothing moves for it: t past the end,
// or padding in the scatter. Padding (a negative id) makes the gather read slot 0, as the torch
// path does (core/everserve/state/mirror.py:579). A block-table gather also writes the slot id.
template <int D, int I>
__device__ __forceinline__ int64_t slot_offset(const RowsArgs& a, uint32_t layer, int64_t t,
                                               int64_t entry) {
  if (t >= a.n) return -1;
  if (I == kByBlocks) {
    // row t is offset t % bs of the (t / bs)-th listed block: no slot id to split again
    const int64_t q = block_of(t, a);
    const int64_t r = t - q * a.bs;
    const int64_t blk = entry;
    if (a.slots_out != nullptr && layer == 0) a.slots_out[t] = blk * a.bs + r;
    if (blk < 0) return D == kGather ? 0 : -1;  // as a negative slot id
    return blk * a.sb + r * a.so;
  }
  int64_t s = entry;
  if (s < 0) s = (D == kGather) ? 0 : -1;
  return s >= 0 ? block_of(s, a) * a.sb + offset_in_block(s, a) * a.so : -1;
}

// Where word v of a tile lies: head index h within the tile's group, slot tl within the tile,
// K or V (k) and word j of the half-row.
struct WordAt {
  uint32_t h, tl, k, j;
};

template <int kOrder>
__device__ __forceinline__ WordAt word_at(const RowsArgs& a, uint32_t v) {
  WordAt w;
  uint32_t q, q2;
  a.div_w.divmod(v, q, w.j);
  if (kOrder == 0) {
    // v = ((k * TS + tl) * HG + h) * W + j
    a.div_h.divmod(q, q2, w.h);
    a.div_ts.divmod(q2, w.k, w.tl);
  } else {
    // v = ((h * TS + tl) * 2 + k) * W + j: K then V of one staged row, row after row
    w.k = q & 1u;
    a.div_ts.divmod(q >> 1, w.h, w.tl);
  }
  return w;
}

// Byte offset of a word of staged row `row` in the layer's part of the staging buffer.
__device__ __forceinline__ int64_t staged_offset(const RowsArgs& a, uint32_t h0, int64_t row,
                                                 const WordAt& w, int64_t word_bytes) {
  return (static_cast<int64_t>(h0 + w.h) * a.cap + row) * (2 * a.half_bytes) +
         w.k * a.half_bytes + static_cast<int64_t>(w.j) * word_bytes;
}

// Move one tile's words: the slots' offsets and the heads' are in LDS, and for the pair scatter
// the staged rows'.
template <typename T, int D, int I>
__device__ __forceinline__ void move_tile(const RowsArgs& a, const int64_t* s_slot,
                                          const int64_t* s_head, const int64_t* s_src,
                                          int64_t layer_base, uint32_t layer, uint32_t group,
                                          int64_t t0) {
  const uint32_t h0 = group * a.HG;
  const int tid = threadIdx.x;
  char* cache_w = reinterpret_cast<char*>(layer_base);
  char* rows_l = a.rows + static_cast<int64_t>(layer) * a.H * a.cap * (2 * a.half_bytes);

  constexpr int kThreads = threads_of(D, I);
  char* sink = reinterpret_cast<char*>(g_sink + (blockIdx.x % kSinkCopies) * kSinkWords) +
               tid * sizeof(u32x4);
  constexpr int kVpt = vpt_of(D, I);
  for (uint32_t v0 = 0; v0 < a.tile_words; v0 += kThreads * kVpt) {
    T w[kVpt];
    const char* src[kVpt];
    char* dst[kVpt];
    bool live[kVpt];
#pragma unroll
    for (int i = 0; i < kVpt; i++) {
      const uint32_t v = v0 + i * kThreads + tid;
      const WordAt at = word_at<word_order(D, I)>(a, v);
      const bool in_tile = v < a.tile_words && h0 + at.h < static_cast<uint32_t>(a.H);
      const int64_t slot_off = in_tile ? s_slot[at.tl] : -1;
      char* cache = cache_w + slot_off + s_head[in_tile ? at.h : 0] + at.k * a.skv + at.j * a.sj;
      const int64_t row = I == kByPairs ? s_src[at.tl] : t0 + at.tl;
      char* staged = rows_l + staged_offset(a, h0, row, at, sizeof(T));
      char* cell = sink + i * kThreads * sizeof(u32x4);
      live[i] = slot_off >= 0;
      src[i] = live[i] ? (D == kGather ? cache : staged) : cell;
      dst[i] = live[i] ? (D == kGather ? staged : cache) : cell;
    }
    if (D == kGather) {
      // Each load stays where it is issued (the scheduler otherwise issued the second word's
      // load first, after the first's address work, so the first store waited for both loads):
      // now the first word's store waits for its own load only. 9-11 interleaved rounds on two
      // boxes: C2 6,110-6,113 against 6,096-6,098 GB/s, C3 6,159 against 6,124, one bf16 head
      // 6,266 against 6,197, the combined layout 6,090 against 6,057, blocks_first unchanged.
#pragma unroll
      for (int i = 0; i < kVpt; i++) {
        w[i] = load_word<T, (nt_of(D, I) & 1) != 0>(src[i]);
        __builtin_amdgcn_sched_barrier(0);
      }
#pragma unroll
      for (int i = 0; i < kVpt; i++)
        store_word<T, (nt_of(D, I) & 2) != 0, EVS_GATHER_STORE_SC1 != 0>(dst[i], w[i]);
    } else {
#pragma unroll
      for (int i = 0; i < kVpt; i++)
        if (live[i]) w[i] = load_word<T, (nt_of(D, I) & 1) != 0>(src[i]);
#pragma unroll
      for (int i = 0; i < kVpt; i++)
        if (live[i]) store_word<T, (nt_of(D, I) & 2) != 0>(dst[i], w[i]);
    }
  }
}

// Fill a tile's slot and head offsets into LDS. The first wave reads both index entries before it
// uses either, so that the two reads are in flight together; its lanes past the tile's slots and
// heads read the tile's last entry again, so that the reads touch only the tile's own lines.
template <int D, int I>
__device__ __forceinline__ void tile_offsets(const RowsArgs& a, const TileId& id, int64_t t0,
                                             int64_t* s_slot, int64_t* s_head, int64_t* s_src) {
  const int tid = threadIdx.x;
  const int h0 = static_cast<int>(id.group) * a.HG;
  static_assert(kMaxTileSlots == 64, "the first wave fills a tile's slots: one lane a slot");
  if (tid < kMaxTileSlots) {
    const int64_t t = t0 + (tid < a.TS ? tid : a.TS - 1);
    // a slot, or a block; the range path reads as a wave, the others a lane at a time
    int64_t entry;
    if constexpr (I == kByRanges)
      entry = wave_slot_in_ranges(a, t0, t < a.n ? t : a.n - 1);
    else
      entry = index_entry<I == kByPairs ? kBySlots : I>(a, t);
    const int64_t src = I == kByPairs ? a.rows_of[t < a.n ? t : a.n - 1] : 0;
    const int hc = h0 + (tid < a.HG ? tid : a.HG - 1);
    const int64_t head = a.heads[hc < a.H ? hc : a.H - 1];
    if (tid < a.TS) {
      int64_t off = slot_offset<D, I == kByBlocks ? kByBlocks : kBySlots>(a, id.layer, t0 + tid,
                                                                          entry);
      if (I == kByPairs) {
        if (src < 0 || src >= a.cap) off = -1;  // a staged row outside the buffer moves nothing
        s_src[tid] = src;
      }
      s_slot[tid] = off;
    }
    if (tid < a.HG && h0 + tid < a.H) s_head[tid] = head * a.sh;
  }
  for (int h = kMaxTileSlots + tid; h < a.HG && h0 + h < a.H; h += threads_of(D, I))
    s_head[h] = a.heads[h0 + h] * a.sh;
}

// One tile per workgroup.
template <typename T, int D, int I>
__global__ __launch_bounds__(threads_of(D, I)) void move_rows(RowsArgs a) {
  __shared__ int64_t s_slot[kMaxTileSlots];  // byte offset of a slot's row in a layer, -1: none
  __shared__ int64_t s_head[kMaxHeads];      // byte offset of a head slot in a row group
  __shared__ int64_t s_src[I == kByPairs ? kMaxTileSlots : 1];  // kByPairs: staged row of a slot

  const TileId id = tile_id(a, xcd_tile(blockIdx.x, gridDim.x, a.xcd_chunk));
  const int64_t t0 = static_cast<int64_t>(id.tile) * a.TS;
  // Read before the block-table path's slot-tag store below: after a store the compiler cannot
  // keep this uniform read scalar (the store might alias it), and a vector read of it made every
  // pass wait for all memory operations in flight (measured 8 % slower).
  const int64_t layer_base = a.layer_ptrs[id.layer];
  tile_offsets<D, I>(a, id, t0, s_slot, s_head, s_src);
  __syncthreads();
  move_tile<T, D, I>(a, s_slot, s_head, s_src, layer_base, id.layer, id.group, t0);
}

struct RowsCall {
  const int64_t* layer_ptrs;
  int64_t L;
  const int64_t* slots;
  const int32_t* blocks;
  int64_t n_index;  // slots, or blocks
  const int64_t* heads;
  int64_t H;
  char* rows;
  int64_t cap;
  int64_t d;
  int64_t bs;
  const int64_t* strides;
  int64_t elem;
  int64_t* slots_out;
  const int64_t* rows_of;
  hipStream_t stream;
  const int64_t* starts = nullptr;      // kByRanges
  const int64_t* first_rows = nullptr;  // kByRanges
  int64_t nranges = 0;                  // kByRanges
};

template <int D, int I, typename T>
int launch_typed(RowsArgs a, int64_t L, uint32_t W, hipStream_t stream, const char* name) {
  const int64_t target = I == kByPairs ? EVS_PAIRS_TILE_WORDS
                         : D == kGather ? EVS_GATHER_TILE_WORDS : EVS_SCATTER_TILE_WORDS;
  const int hpt = I == kByPairs ? EVS_PAIRS_HEADS_PER_TILE
                  : D == kGather ? EVS_GATHER_HEADS_PER_TILE : EVS_SCATTER_HEADS_PER_TILE;
  a.HG = (hpt > 0 && hpt < a.H) ? hpt : a.H;
  a.group_fastest = D == kGather      ? EVS_GATHER_GROUP_FASTEST
                    : I == kByRanges ? EVS_RANGES_GROUP_FASTEST
                                     : EVS_SCATTER_GROUP_FASTEST;
  a.xcd_chunk = I == kByPairs ? EVS_PAIRS_XCD_CHUNK
                : I == kByRanges ? EVS_RANGES_XCD_CHUNK
                : D == kGather ? EVS_GATHER_XCD_CHUNK : EVS_SCATTER_XCD_CHUNK;
  const int64_t groups = (a.H + a.HG - 1) / a.HG;
  if (D == kGather && I != kByPairs && groups == 1) a.xcd_chunk = EVS_GATHER_XCD_CHUNK_ONE_GROUP;
  const int64_t per_slot = static_cast<int64_t>(a.HG) * 2 * W;
  int64_t ts = target / per_slot;
  ts = ts < 1 ? 1 : (ts > kMaxTileSlots ? kMaxTileSlots : ts);
  if (ts > a.n) ts = a.n;
  const int64_t tiles = (a.n + ts - 1) / ts;
  const int64_t grid = tiles * groups * L;
  EVS_REQUIRE(ts * per_slot < (int64_t{1} << 31), "%s: a tile of %lld words is too large", name,
              static_cast<long long>(ts * per_slot));
  // HIP on AMD GPUs takes at most 2^32 - 1 work-items along x (gridDim.x * blockDim.x)
  EVS_REQUIRE(grid * threads_of(D, I) < (int64_t{1} << 32),
              "%s: %lld workgroups of %d threads exceed the launch limit of 2^32 - 1 work-items; "
              "split the call by layers", name, static_cast<long long>(grid), threads_of(D, I));
  a.TS = static_cast<int>(ts);
  a.tile_words = static_cast<uint32_t>(ts * per_slot);
  a.div_w = FastDiv(W);
  a.div_h = FastDiv(static_cast<uint32_t>(a.HG));
  a.div_ts = FastDiv(static_cast<uint32_t>(ts));
  a.div_tiles = FastDiv(static_cast<uint32_t>(tiles));
  a.div_groups = FastDiv(static_cast<uint32_t>(groups));
  hipLaunchKernelGGL((move_rows<T, D, I>), dim3(static_cast<uint32_t>(grid)),
                     dim3(threads_of(D, I)), 0, stream, a);
  EVS_LAUNCHED(name);
  return EVS_OK;
}

// The checks of a call's arguments. *moves is false when the call has nothing to move (no slot,
// head or layer); its pointers are not checked then.
template <int D, int I>
int check_call(const RowsCall& c, const char* name, bool* moves) {
  *moves = false;
  EVS_REQUIRE(c.strides != nullptr, "%s: a layout is five strides", name);
  EVS_REQUIRE(c.elem == 1 || c.elem == 2 || c.elem == 4, "%s: unsupported element size %lld",
              name, static_cast<long long>(c.elem));
  EVS_REQUIRE(c.L >= 0 && c.n_index >= 0 && c.H >= 0, "%s: negative count", name);
  EVS_REQUIRE(c.d >= 1 && c.bs >= 1, "%s: head_dim and block_size must be positive", name);
  EVS_REQUIRE(c.H <= kMaxHeads, "%s: at most %d head slots per call, got %lld", name, kMaxHeads,
              static_cast<long long>(c.H));
  const int64_t n = I == kByBlocks ? c.n_index * c.bs : c.n_index;
  // a pair names its staged row, so pairs may outnumber the rows (a row written to several slots)
  EVS_REQUIRE(I == kByPairs || n <= c.cap,
              "%s: more slots (%lld) than the staging capacity (%lld)", name,
              static_cast<long long>(n), static_cast<long long>(c.cap));
  EVS_REQUIRE(c.cap >= 0, "%s: negative capacity", name);
  if (n == 0 || c.H == 0 || c.L == 0) return EVS_OK;
  EVS_REQUIRE(c.layer_ptrs != nullptr && c.heads != nullptr && c.rows != nullptr,
              "%s: null pointer", name);
  EVS_REQUIRE(I == kByBlocks ? c.blocks != nullptr
              : I == kByRanges ? c.starts != nullptr && c.first_rows != nullptr
                               : c.slots != nullptr,
              "%s: null index", name);
  EVS_REQUIRE(I != kByPairs || c.rows_of != nullptr, "%s: null row list", name);
  EVS_REQUIRE(I != kByRanges || c.nranges >= 1, "%s: rows to move but no range", name);
  *moves = true;
  return EVS_OK;
}

template <int D, int I>
int move(const RowsCall& c, const char* name) {
  bool moves = false;
  const int rc = check_call<D, I>(c, name, &moves);
  if (rc != EVS_OK || !moves) return rc;
  const int64_t n = I == kByBlocks ? c.n_index * c.bs : c.n_index;
  const int64_t e = c.elem;
  RowsArgs a{};
  a.layer_ptrs = c.layer_ptrs;
  a.slots = c.slots;
  a.blocks = c.blocks;
  a.heads = c.heads;
  a.rows = c.rows;
  a.slots_out = c.slots_out;
  a.rows_of = c.rows_of;
  a.starts = c.starts;
  a.first_rows = c.first_rows;
  a.nranges = c.nranges;
  a.n = n;
  a.cap = c.cap;
  a.half_bytes = c.d * e;
  a.sb = c.strides[0] * e;
  a.so = c.strides[1] * e;
  a.sh = c.strides[2] * e;
  a.skv = c.strides[3] * e;
  a.bs = c.bs;
  a.bs_shift = -1;
  if ((c.bs & (c.bs - 1)) == 0) {
    int s = 0;
    while ((int64_t{1} << s) < c.bs) ++s;
    a.bs_shift = s;
  }
  a.H = static_cast<int>(c.H);

  const bool vectors = c.strides[4] == 1 && aligned16(c.d * e) &&
                       aligned16(reinterpret_cast<int64_t>(c.rows)) && aligned16(a.sb) &&
                       aligned16(a.so) && aligned16(a.sh) && aligned16(a.skv);
  if (vectors) {
    a.sj = 16;
    return launch_typed<D, I, u32x4>(a, c.L, static_cast<uint32_t>(c.d * e / 16), c.stream, name);
  }
  a.sj = c.strides[4] * e;
  EVS_REQUIRE(c.d < (int64_t{1} << 24), "%s: head_dim too large", name);
  switch (e) {
    case 1:
      return launch_typed<D, I, uint8_t>(a, c.L, static_cast<uint32_t>(c.d), c.stream, name);
    case 2:
      return launch_typed<D, I, uint16_t>(a, c.L, static_cast<uint32_t>(c.d), c.stream, name);
    default:
      return launch_typed<D, I, uint32_t>(a, c.L, static_cast<uint32_t>(c.d), c.stream, name);
  }
}

}  // namespace
}  // namespace evs

extern "C" int evs_gather_rows(const int64_t* layer_ptrs, int64_t num_layers,
                               const int64_t* slots, int64_t num_slots, const int64_t* heads,
                               int64_t num_heads, void* out, int64_t capacity, int64_t head_dim,
                               int64_t block_size, const int64_t* strides, int64_t elem_size,
                               void* stream) {
  evs::clear_error();
  evs::RowsCall c{layer_ptrs, num_layers, slots, nullptr, num_slots, heads, num_heads,
                  static_cast<char*>(out), capacity, head_dim, block_size, strides, elem_size,
                  nullptr, nullptr, evs::as_stream(stream)};
  return evs::move<evs::kGather, evs::kBySlots>(c, "evs_gather_rows");
}

extern "C" int evs_gather_blocks(const int64_t* layer_ptrs, int64_t num_layers,
                                 const int32_t* block_ids, int64_t num_blocks,
                                 const int64_t* heads, int64_t num_heads, void* out,
                                 int64_t capacity, int64_t head_dim, int64_t block_size,
                                 const int64_t* strides, int64_t elem_size, int64_t* slots_out,
                                 void* stream) {
  evs::clear_error();
  evs::RowsCall c{layer_ptrs, num_layers, nullptr, block_ids, num_blocks, heads, num_heads,
                  static_cast<char*>(out), capacity, head_dim, block_size, strides, elem_size,
                  slots_out, nullptr, evs::as_stream(stream)};
  return evs::move<evs::kGather, evs::kByBlocks>(c, "evs_gather_blocks");
}

extern "C" int evs_scatter_rows(const int64_t* layer_ptrs, int64_t num_layers,
                                const int64_t* slots, int64_t num_slots, const int64_t* heads,
                                int64_t num_heads, const void* in, int64_t capacity,
                                int64_t head_dim, int64_t block_size, const int64_t* strides,
                                int64_t elem_size, void* stream) {
  evs::clear_error();
  evs::RowsCall c{layer_ptrs, num_layers, slots, nullptr, num_slots, heads, num_heads,
                  const_cast<char*>(static_cast<const char*>(in)), capacity, head_dim,
                  block_size, strides, elem_size, nullptr, nullptr, evs::as_stream(stream)};
  return evs::move<evs::kScatter, evs::kBySlots>(c, "evs_scatter_rows");
}

extern "C" int evs_scatter_pairs(const int64_t* layer_ptrs, int64_t num_layers,
                                 const int64_t* slots, const int64_t* rows_of, int64_t num_pairs,
                                 const int64_t* heads, int64_t num_heads, const void* in,
                                 int64_t capacity, int64_t head_dim, int64_t block_size,
                                 const int64_t* strides, int64_t elem_size, void* stream) {
  evs::clear_error();
  evs::RowsCall c{layer_ptrs, num_layers, slots, nullptr, num_pairs, heads, num_heads,
                  const_cast<char*>(static_cast<const char*>(in)), capacity, head_dim,
                  block_size, strides, elem_size, nullptr, rows_of, evs::as_stream(stream)};
  return evs::move<evs::kScatter, evs::kByPairs>(c, "evs_scatter_pairs");
}

extern "C" int evs_scatter_ranges(const int64_t* layer_ptrs, int64_t num_layers,
                                  const int64_t* starts, const int64_t* first_rows,
                                  int64_t num_ranges, int64_t num_rows, const int64_t* heads,
                                  int64_t num_heads, const void* in, int64_t capacity,
                                  int64_t head_dim, int64_t block_size, const int64_t* strides,
                                  int64_t elem_size, void* stream) {
  evs::clear_error();
  EVS_REQUIRE(num_ranges >= 0, "evs_scatter_ranges: negative range count");
  evs::RowsCall c{layer_ptrs, num_layers, nullptr, nullptr, num_rows, heads, num_heads,
                  const_cast<char*>(static_cast<const char*>(in)), capacity, head_dim,
                  block_size, strides, elem_size, nullptr, nullptr, evs::as_stream(stream),
                  starts, first_rows, num_ranges};
  return evs::move<evs::kScatter, evs::kByRanges>(c, "evs_scatter_ranges");
}
