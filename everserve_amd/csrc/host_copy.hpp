// Host-memory copies with nontemporal stores, for the library's host copies (the restore's host
// gather, the store's commit). A plain store first reads every line it writes into the cache;
// where the destination is cold (a pinned buffer the DMA engine reads next, a table row at a
// random place in gigabytes of tables) that read is a third stream of memory traffic or a
// cache miss per line. Nontemporal stores are weakly ordered: the thread that made them calls
// stream_fence() before anyone learns that the copy is done.
#pragma once

#include <cstddef>
#include <cstdint>
#include <cstring>

namespace evs {

typedef long long v2i64 __attribute__((ext_vector_type(2)));

// memcpy with 16-byte nontemporal stores where dst is 16-byte aligned; plain copies for the
// unaligned head and the tail.
inline void stream_copy(char* dst, const char* src, size_t bytes) {
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

// Drains this thread's nontemporal stores.
inline void stream_fence() {
#if defined(__x86_64__)
  __builtin_ia32_sfence();
#else
  __atomic_thread_fence(__ATOMIC_SEQ_CST);
#endif
}

}  // namespace evs
