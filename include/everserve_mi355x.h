/*
 * everserve_mi355x.h — the C ABI of libeverserve_mi355x.so, the MI355X (gfx950) per-worker KV
 * data path: the step's KV snapshot gather, the restore scatter, and the reduction stage of the
 * failure-detecting all-reduce.
 *
 * Every entry point returns 0 on success and a nonzero EVS_E* code on failure; evs_last_error()
 * then gives a message for the calling thread. Pointers named "device" are addresses in the
 * current HIP device's address space (HBM, or host memory mapped into it); `stream` is a
 * hipStream_t passed as void* (NULL is the null stream). Nothing here allocates on the hot path
 * (the gathers, the scatter and the reductions), and nothing here synchronises a stream: every
 * kernel is enqueued on `stream` and the call returns.
 *
 * The reference exposes the same surface as the pybind module `everserve_kernels`
 * (core/csrc/kernels.cpp:9-31, declared at core/csrc/kernels.h:18-59); each declaration below
 * names the reference entry it replaces.
 */
#ifndef EVERSERVE_MI355X_H
#define EVERSERVE_MI355X_H

#include <stddef.h>
#include <stdint.h>

#ifdef __cplusplus
extern "C" {
#endif

/* Return codes. */
#define EVS_OK 0
#define EVS_EINVAL 1 /* a precondition failed; nothing was enqueued */
#define EVS_EHIP 2   /* a HIP runtime call failed */

/* The slot region's layout shared with the Python side (core/csrc/kernels.h:18-22: kMaxRows,
 * kCtrlWords, kAbort, kLate, kBound). A region is MAX_ROWS control rows of CTRL_WORDS int64
 * words; word ABORT releases a waiting reduction, word LATE receives the mask of the rows a
 * reduction waits for past the bound, word BOUND holds that bound in nanoseconds (0 = off). */
#define EVS_MAX_ROWS 8
#define EVS_CTRL_WORDS 16
#define EVS_ABORT 1
#define EVS_LATE 11
#define EVS_BOUND 12

/* The local reduction's status word (evs_local_reduce, state[0]) once a call has finished:
 * (epoch << 16) | (reason << 8) | late_mask, reason EVS_REDUCE_DONE or the bits below that
 * apply (workgroups whose waits ended differently contribute each their own). */
#define EVS_REDUCE_DONE 0      /* every member's flag carried the call's epoch */
#define EVS_REDUCE_ABORTED 1   /* released by the ABORT control word */
#define EVS_REDUCE_TIMED_OUT 2 /* the hard timeout passed with members still missing */
#define EVS_REDUCE_BAD_ORDER 4 /* `order` named a row outside [0, EVS_MAX_ROWS): that position
                                  added nothing, and the call did not wait for it */
#define EVS_REDUCE_STATE_WORDS 288 /* state[0] the outcome; the rest the kernel's counters */

/* The message of the last failed call on this thread ("" if none). */
const char* evs_last_error(void);

/* The layout constants above as the library was built with them: out[0..4] = MAX_ROWS,
 * CTRL_WORDS, ABORT, LATE, BOUND. The Python shim exports them as the reference module's
 * attributes (core/csrc/kernels.cpp:12-16), which core/everserve/comm/slotkernel.py:98-120
 * compares against its own copy. `n` must be at least 5. */
int evs_layout_constants(int64_t* out, int64_t n);

/* Copy one step's K and V rows of every layer and held head slot into a staging buffer laid out
 * [num_layers, num_heads, capacity, 2, head_dim] (elements of elem_size bytes), on `stream`.
 * Replaces gather_rows (core/csrc/gather.cu:100-135, kernels.h:27-29). For t < num_slots:
 *
 *   out[l][h][t][k][j] = layer_l[(s / block_size) * strides[0] + (s % block_size) * strides[1]
 *                                + heads[h] * strides[2] + k * strides[3] + j * strides[4]]
 *   with s = max(slots[t], 0)   (a negative slot id is padding and reads slot 0)
 *
 * strides (host array of five, in elements) are the cache layout's block, offset-in-block, head
 * slot, K-or-V and element strides (core/everserve/state/kvcopy.py:105-116). layer_ptrs (device,
 * num_layers int64 addresses), slots (device, int64) and heads (device, int64) are read by the
 * kernel; rows num_slots..capacity-1 are not written. Bytes move unchanged, so fp8 (e4m3/e5m2)
 * caches go through elem_size 1 bit-exactly. Requires elem_size in {1, 2, 4} and
 * num_slots <= capacity; returns EVS_OK with nothing enqueued when any count is zero. The 16-byte
 * path is taken when strides[4] == 1 and head_dim*elem_size, out and every other stride (in bytes)
 * are multiples of 16; the caller guarantees the layer bases are 16-byte aligned then, as the
 * reference's caller does (core/everserve/state/mirror.py:344). */
int evs_gather_rows(const int64_t* layer_ptrs, int64_t num_layers, const int64_t* slots,
                    int64_t num_slots, const int64_t* heads, int64_t num_heads, void* out,
                    int64_t capacity, int64_t head_dim, int64_t block_size,
                    const int64_t* strides, int64_t elem_size, void* stream);

/* evs_gather_rows over whole blocks of a block table: the rows equal those of evs_gather_rows
 * with slots[t] = block_ids[t / block_size] * block_size + t % block_size, t < num_blocks *
 * block_size. When slots_out is not NULL the kernel also writes those slot ids there (device,
 * int64, num_blocks * block_size): the step descriptor's sequence tags
 * (proto/everserve/proto/mirror.proto:50-51). Replaces the host-side expansion of the staged
 * block ids (core/everserve/reference/staging.py:51-94 chooses them) followed by gather_rows. */
int evs_gather_blocks(const int64_t* layer_ptrs, int64_t num_layers, const int32_t* block_ids,
                      int64_t num_blocks, const int64_t* heads, int64_t num_heads, void* out,
                      int64_t capacity, int64_t head_dim, int64_t block_size,
                      const int64_t* strides, int64_t elem_size, int64_t* slots_out,
                      void* stream);

/* The inverse of evs_gather_rows: write rows laid out [num_layers, num_heads, capacity, 2,
 * head_dim] back into the paged caches at slots[t] and head slots heads[h]. A negative slot is
 * padding and is skipped (nothing written). Slots must be distinct (a restore's written slot
 * ranges are, store/src/storage.rs:430-451); with duplicates which row lands is unspecified.
 * One kernel, rows read in staged order, nothing allocated. For a restore that writes a whole
 * cache through a permuted block table, evs_order_pairs then evs_scatter_pairs write the same
 * bytes in slot order, faster (the shipped loader's scatter_rows does so from 2^18 slots and
 * 8 GiB of rows, in a workspace it keeps). Replaces the restore's per-table PagedKV.write_rows
 * scatter (core/everserve/state/mirror.py:926-937, core/everserve/state/kvcopy.py:118-128). */
int evs_scatter_rows(const int64_t* layer_ptrs, int64_t num_layers, const int64_t* slots,
                     int64_t num_slots, const int64_t* heads, int64_t num_heads, const void* in,
                     int64_t capacity, int64_t head_dim, int64_t block_size,
                     const int64_t* strides, int64_t elem_size, void* stream);

/* The scatter by (slot, staged row) pairs: for every listed i, layer and head index h, write staged
 * row rows_of[i] of [num_layers, num_heads, capacity, 2, head_dim] into the cache at slot slots[i]
 * and head slot heads[h]. evs_scatter_rows is the case rows_of[i] = i. A negative slot, or a row
 * outside [0, capacity), moves nothing. The kernel writes in listed order, all heads of a slot
 * together, so a caller that lists its slots in increasing order writes each layer's cache front
 * to back; for a restore into a cache whose block table is a permutation of the staged order
 * (the spare's fresh cache) that is the faster order. Slots must be distinct, as for
 * evs_scatter_rows. No counterpart in the reference: it is the restore's scatter
 * (core/everserve/state/mirror.py:926-937) with the order of its writes chosen by the caller. */
int evs_scatter_pairs(const int64_t* layer_ptrs, int64_t num_layers, const int64_t* slots,
                      const int64_t* rows_of, int64_t num_pairs, const int64_t* heads,
                      int64_t num_heads, const void* in, int64_t capacity, int64_t head_dim,
                      int64_t block_size, const int64_t* strides, int64_t elem_size,
                      void* stream);

/* The scatter of written ranges: staged row t of [num_layers, num_heads, capacity, 2, head_dim]
 * goes to slot starts[k] + (t - first_rows[k]), for the range k with first_rows[k] <= t <
 * first_rows[k + 1], t < num_rows, at head slots heads[h]. starts (num_ranges entries) and
 * first_rows (num_ranges + 1: first_rows[0] = 0, ascending, the last one num_rows) are device
 * arrays; an empty range is passed over. This is evs_scatter_rows with the slots given as the
 * store's (start, count) ranges (proto/everserve/proto/mirror.proto:102-117) instead of one id a
 * row: no slot array to build or copy. With the ranges ascending, as a restore's are
 * (store/src/storage.rs:430-451), the writes run through each layer's cache front to back and the
 * launch deals each XCD a contiguous part of them. Replaces the restore's per-table
 * PagedKV.write_rows of a table's written ranges (core/everserve/state/mirror.py:926-937). */
int evs_scatter_ranges(const int64_t* layer_ptrs, int64_t num_layers, const int64_t* starts,
                       const int64_t* first_rows, int64_t num_ranges, int64_t num_rows,
                       const int64_t* heads, int64_t num_heads, const void* in, int64_t capacity,
                       int64_t head_dim, int64_t block_size, const int64_t* strides,
                       int64_t elem_size, void* stream);

/* The pairs for evs_scatter_pairs in slot order, on the device, for a caller whose slot list is
 * in HBM: slots_out[i] = slots[rows_out[i]], by increasing slot, where rows_out is a permutation
 * of 0..num_pairs-1 (stable: equal slots keep their listed order). Only the low key_bits bits of
 * a slot id are compared (1..64; at least the bits of the cache's largest slot id); a negative
 * slot id (padding) lands wherever its low bits put it, and evs_scatter_pairs skips it.
 * `workspace` is device memory of at least evs_order_pairs_workspace(num_pairs, key_bits) bytes,
 * 256-byte aligned, owned by the caller; the call allocates nothing and does not synchronise.
 * The sort clears its own counters in the workspace with hipMemsetAsync, so keep this call out
 * of captured HIP graphs. num_pairs < 2^31. No counterpart in the reference: it orders the restore's writes (see
 * evs_scatter_pairs); the host-side equivalent is everserve_amd.state.restore.destination_order. */
int evs_order_pairs_workspace(int64_t num_pairs, int key_bits, int64_t* bytes);
int evs_order_pairs(const int64_t* slots, int64_t num_pairs, int key_bits, int64_t* slots_out,
                    int64_t* rows_out, void* workspace, int64_t workspace_bytes, void* stream);

/* evs_order_pairs without a workspace argument, for callers that cannot allocate device memory
 * (tight serving loops, harnesses that forbid hipMalloc). Not for HIP graph capture: see the
 * memset below. No counterpart in the reference. Its scratch is a file-scope device array of
 * EVS_ORDER_STATIC_SCRATCH_BYTES that every GPU the library runs on holds until the process ends;
 * num_pairs is at most EVS_ORDER_STATIC_MAX_PAIRS (a larger call is refused with a message, and
 * nothing is enqueued). Calls on one GPU share that GPU's array: two calls that overlap on one GPU
 * (on different streams, or from different threads) race and give wrong results, so order them.
 * The call allocates nothing and does not synchronise; like evs_order_pairs, rocPRIM clears its
 * counters with hipMemsetAsync, so keep it out of captured graphs. */
#define EVS_ORDER_STATIC_MAX_PAIRS (1 << 20)
#define EVS_ORDER_STATIC_SCRATCH_BYTES (32 << 20)
int evs_order_pairs_static(const int64_t* slots, int64_t num_pairs, int key_bits,
                           int64_t* slots_out, int64_t* rows_out, void* stream);

/* The reduction stage of the failure-detecting all-reduce over member buffers already in this
 * GPU's HBM (the local stage of core/csrc/slot.cu:118-224):
 *
 *   out[i] = bf16_rne( ((0.0f + f32(x_{o1}[i])) + f32(x_{o2}[i])) + ... )
 *
 * with o = order[1 .. order[0]] (device int32 [1 + EVS_MAX_ROWS], rows < EVS_MAX_ROWS),
 * x_r = the bf16 buffer at bufs[r] (device table of EVS_MAX_ROWS int64 addresses) and bf16_rne
 * torch's round to nearest even (NaN becomes 0x7FC0), i < n. Member r's payload is ready when
 * flags[r] (device uint64 [EVS_MAX_ROWS]) equals `epoch`; the kernel waits for every member's flag
 * before it reads that member. The wait is bounded: it ends when the ABORT word of `ctrl` (an
 * EVS_CTRL_WORDS int64 row, host-mapped or device) is nonzero, or when timeout_ns has passed
 * (timeout_ns <= 0 means 1 s); a member still missing then contributes zeros. While waiting past
 * ctrl[EVS_BOUND] ns (0 = off), the kernel writes the mask of the rows it waits for into
 * ctrl[EVS_LATE], and the last block that named clears it when its wait ends. `state` (device
 * uint64 [EVS_REDUCE_STATE_WORDS], zeroed once before first use) receives in state[0], when the
 * call finishes, (epoch << 16) | (reason << 8) | late_mask with reason as above; the
 * other words are the kernel's own and return to zero at the end of every call, so a captured
 * HIP graph can replay it. Requires 0 <= n; out and every member buffer 2-byte aligned (16-byte
 * aligned takes the vector path). */
int evs_local_reduce(const int64_t* bufs, const uint64_t* flags, const int32_t* order, void* out,
                     int64_t n, uint64_t epoch, int64_t timeout_ns, int64_t* ctrl,
                     uint64_t* state, void* stream);

/* The slot collective: sum bf16 `inp` (n elements, even, n <= maxn) over the members `order`
 * lists, in that order, into `out`, on `stream`. Replaces slot_all_reduce (core/csrc/slot.cu:
 * 234-281, kernels.h:43-45) argument for argument, plus num_seqs and timeout_ns:
 *   bufs      device table of EVS_MAX_ROWS addresses, each row's word buffer: [2][maxn/2]
 *             uint64 words (pull) or [2][EVS_MAX_ROWS][maxn/2] (push);
 *   ctrl      device address of the region's control rows (EVS_MAX_ROWS x EVS_CTRL_WORDS int64);
 *             row `row`'s ABORT and BOUND are read, its LATE written;
 *   order     device int32 [1 + EVS_MAX_ROWS] = [count, rows...];
 *   seqs      device int64 [num_seqs], num_seqs > evs_slot_blocks(maxn, 1): a sequence counter
 *             per workgroup, then the count of workgroups that named a late member; zeroed at a
 *             membership change (core/everserve/comm/slotkernel.py:713-727);
 *   words     8-byte words per thread: 1, 2, 4, 8 or 16; push nonzero for the push variant.
 * A word is (sequence << 32) | two bf16. The wait ends when every member's words carry the
 * call's sequence number, at the ABORT word, or after timeout_ns (<= 0: 30 s; the reference waits
 * for ABORT alone); a member's missing words then sum as zeros. */
int evs_slot_all_reduce(const void* inp, void* out, int64_t n, const int64_t* bufs, int64_t* ctrl,
                        const int32_t* order, int64_t* seqs, int64_t num_seqs, int64_t row,
                        int64_t maxn, int64_t words, int push, int64_t timeout_ns, void* stream);

/* Sequence counters the slot collective needs for tensors of up to `maxn` elements at `words`
 * eight-byte words per thread: ceil((maxn / 2) / (256 * words)). Replaces slot_blocks
 * (core/csrc/slot.cu:229-232). Writes the count to *out. */
int evs_slot_blocks(int64_t maxn, int64_t words, int64_t* out);

/* Pin `bytes` of host memory at `ptr`, mapped into the device address space; *device_ptr receives
 * the address kernels use. Replaces host_register_mapped (core/csrc/gather.cu:137-144). */
int evs_host_register_mapped(void* ptr, int64_t bytes, void** device_ptr);

/* Undo evs_host_register_mapped. Replaces host_unregister (core/csrc/gather.cu:146-148). */
int evs_host_unregister(void* ptr);

/* Pinned, coherent host memory mapped into the device, allocated by the runtime (for hosts where
 * registering existing memory is not allowed): *host_ptr and *device_ptr receive the two views.
 * No reference counterpart; it stands in for host_register_mapped where that is refused. */
int evs_host_alloc_mapped(int64_t bytes, void** host_ptr, void** device_ptr);
int evs_host_free(void* host_ptr);

/* Device memory outside any caching allocator, zeroed before return. Replaces device_alloc and
 * device_free (core/csrc/slot.cu:283-290). */
int evs_device_alloc(int64_t bytes, void** ptr);
int evs_device_free(void* ptr);

/* Zero `bytes` of device memory on `stream` with a fill kernel (a graph may capture it). Replaces
 * memset_async (core/csrc/slot.cu:292-295). */
int evs_memset_async(void* ptr, int64_t bytes, void* stream);

/* Copy `groups` runs of `bytes` bytes, run g from src + g * pitch to dst + g * pitch, on `stream`
 * (hipMemcpy2DAsync; one linear copy when bytes == pitch). Direction follows the pointers: the
 * staging buffer's filled rows (num_slots of each (layer, head) run of `capacity`) to pinned host
 * memory, or back. Stands in for the reference's zero-copy writes through a host-mapped staging
 * file (core/everserve/state/mirror.py:349-356,614-622): the gather writes HBM at HBM speed and
 * the copy engine moves the rows over PCIe on the side stream. */
int evs_copy_rows_async(void* dst, const void* src, int64_t groups, int64_t bytes, int64_t pitch,
                        void* stream);

/* The restore's host gather: copy the rows of `nranges` slot ranges (starts[k], counts[k]) of a
 * store table at `src` ([src_rows, row_bytes], a shared-memory mapping) into `dst` (room for
 * dst_rows rows), one range after another, on up to max_threads host threads; *rows_out (if not
 * NULL) receives the row count. Every range must lie within the table and all of them must fit
 * in dst, or nothing is copied. Host memory only, no device call. Replaces the per-table
 * torch.index_select of the restore (core/everserve/state/mirror.py:926-932); the ranges are the
 * table's written SlotRanges (proto/everserve/proto/mirror.proto:102-117). */
int evs_host_gather_ranges(const void* src, int64_t src_rows, int64_t row_bytes,
                           const int64_t* starts, const int64_t* counts, int64_t nranges,
                           void* dst, int64_t dst_rows, int64_t max_threads, int64_t* rows_out);

/* evs_host_gather_ranges over several tables with the same written ranges (the head tables of one
 * layer: a store commit writes every held head of a layer at the same slots): table j's rows land
 * at dst + j * dst_rows * row_bytes, so dst holds num_tables * dst_rows rows. One call, one set of
 * host threads for all of them. Everything is checked before anything is copied. Replaces the
 * per-table torch.index_select of the restore (core/everserve/state/mirror.py:926-932) for a
 * restore that scatters a layer's heads in one launch. */
int evs_host_gather_tables(const void* const* srcs, int64_t num_tables, int64_t src_rows,
                           int64_t row_bytes, const int64_t* starts, const int64_t* counts,
                           int64_t nranges, void* dst, int64_t dst_rows, int64_t max_threads,
                           int64_t* rows_out);

/* Deliver `runs` runs of `run_bytes` bytes from device memory (run g at src + g * src_pitch) into
 * host memory that need not be pinned (run g at dst + g * dst_pitch), such as a staging file in
 * shared memory that the node's store maps by name. The copy engine moves batches of rows on
 * `stream` into two pinned bounce buffers of `bounce_bytes` each (a positive multiple of 64) in
 * turn, while up to max_threads host threads copy the previous batch into dst with nontemporal
 * stores. Blocks the calling thread until every byte is in dst; run it off the step thread. The
 * device rows must be complete before the call (the caller waits for the gather's event).
 * Stands in for the reference's zero-copy writes through a cudaHostRegister'd staging file
 * (core/everserve/state/mirror.py:349-356,588-634) where registering existing memory is not
 * allowed. */
int evs_deliver_rows(void* dst, int64_t dst_pitch, const void* src, int64_t src_pitch,
                     int64_t runs, int64_t run_bytes, void* bounce0, void* bounce1,
                     int64_t bounce_bytes, int64_t max_threads, void* stream);

/* The node store's commit copy (store/src/storage.rs:864-957; copy loop :916-943): the rows of
 * one staged step into `ntables` store tables, on the host.
 *   stage              the staged bytes (stage_bytes long); table k's rows start at
 *                      stage_offsets[k], row t at + t * row_bytes (the StagedStep layout,
 *                      storage.rs:521-540);
 *   tables[k]          table k's rows, [num_slots, row_bytes];
 *   written_step[k]    table k's per-slot step of the last write (uint64 [num_slots]);
 *   crc[k]             table k's per-slot CRC32C of the row as written (uint32 [num_slots]).
 * For each slot id slots[t] >= 0, row t goes to table row slots[t]; runs of consecutive slot ids
 * copy as one memcpy; written_step becomes max(step, 1) and crc the Castagnoli CRC32C of the row
 * (Layer::mark_written, storage.rs:494-504). Negative ids are padding and are skipped. Every slot
 * id and offset is checked before anything is written (a slot >= num_slots refuses the call).
 * Tables are independent and are committed on up to max_threads host threads;
 * *newly_written (if not NULL) receives the slots written for the first time, over all tables.
 * Host memory only, no device call. */
int evs_store_commit(const void* stage, int64_t stage_bytes, const int64_t* stage_offsets,
                     int64_t ntables, void* const* tables, uint64_t* const* written_step,
                     uint32_t* const* crc, int64_t num_slots, int64_t row_bytes,
                     const int64_t* slots, int64_t nslots, uint64_t step, int64_t max_threads,
                     int64_t* newly_written);

/* CRC32C (Castagnoli: reflected polynomial 0x82F63B78, initial value and final xor 0xFFFFFFFF),
 * the checksum the store keeps per row (the crc32c crate, store/Cargo.toml:25): of `bytes` bytes
 * into *out, and of `rows` consecutive rows of row_bytes each into out[0..rows). Host only. */
int evs_crc32c(const void* data, int64_t bytes, uint32_t* out);
int evs_crc32c_rows(const void* data, int64_t row_bytes, int64_t rows, uint32_t* out);

/* Stream-to-stream ordering on one device without a cache writeback. A HIP event records with a
 * system-scope fence by default (the L2 written back and invalidated at the record); ordering one
 * stream's later work after another's on the same device needs none of it, since every kernel
 * releases its writes at its end. On a decode step that fence cost more than the snapshot it
 * ordered (measured: 258 us per step against 14 us for the gather). evs_event_create makes an
 * event with timing off and, unless system_fence is nonzero, without that fence;
 * evs_stream_handoff records it on `producing` and makes `waiting` wait for it. An event a host
 * thread waits on before reading memory a kernel wrote keeps the fence (system_fence = 1). The
 * reference orders its side stream after the forward with a default CUDA event
 * (core/everserve/state/mirror.py:696-697). */
int evs_event_create(int system_fence, void** event);
int evs_event_destroy(void* event);
int evs_event_record(void* event, void* stream);
int evs_event_synchronize(void* event);
int evs_stream_handoff(void* producing, void* waiting, void* event);

/* Inter-process memory handles (64 bytes). Replace ipc_handle, ipc_open and ipc_close
 * (core/csrc/slot.cu:297-312). */
int evs_ipc_handle(void* ptr, uint8_t* handle_out, int64_t handle_bytes);
int evs_ipc_open(const uint8_t* handle, int64_t handle_bytes, void** ptr);
int evs_ipc_close(void* ptr);

/* The current device's wall-clock counter rate in kHz (the clock the bounded waits use). */
int evs_wall_clock_khz(int64_t* khz);

#ifdef __cplusplus
}
#endif

#endif /* EVERSERVE_MI355X_H */
