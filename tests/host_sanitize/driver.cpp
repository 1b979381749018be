// The library's multi-threaded host entry points under AddressSanitizer or ThreadSanitizer, on
// the CPU: evs_store_commit on 16 threads, evs_host_gather_ranges and evs_host_gather_tables on
// 8, evs_crc32c_rows. Each
// result is checked against a plain serial computation here. Built and run by run.sh; host code
// only (the .hip files hold no kernels this driver calls).
#include <cstdint>
#include <cstdio>
#include <cstring>
#include <random>
#include <thread>
#include <vector>
extern "C" {
int evs_store_commit(const void*, int64_t, const int64_t*, int64_t, void* const*, uint64_t* const*,
                     uint32_t* const*, int64_t, int64_t, const int64_t*, int64_t, uint64_t, int64_t,
                     int64_t*);
int evs_host_gather_ranges(const void*, int64_t, int64_t, const int64_t*, const int64_t*, int64_t,
                           void*, int64_t, int64_t, int64_t*);
int evs_host_gather_tables(const void* const*, int64_t, int64_t, int64_t, const int64_t*,
                           const int64_t*, int64_t, void*, int64_t, int64_t, int64_t*);
int evs_crc32c_rows(const void*, int64_t, int64_t, uint32_t*);
int evs_crc32c(const void*, int64_t, uint32_t*);
const char* evs_last_error();
}
// runtime.hip's evs_wall_clock_khz calls this; its definition lives in reduce.hip, which holds
// kernels and is not part of this host-only build
namespace evs { int wall_clock_khz(int64_t* k) { *k = 100000; return 0; } }
static int fails = 0;
#define CHECK(c) do { if (!(c)) { std::printf("FAIL %s:%d %s\n", __FILE__, __LINE__, #c); fails++; } } while (0)

int main() {
  std::mt19937_64 rng(7);
  // store commit: 16 tables x 8192 slots x 512 B, a step of 4096 slots (32 MiB: nontemporal
  // stores) and one of 256 (2 MiB: memcpy, still 16 threads), with runs, padding and a repeat
  for (const int64_t N : {int64_t{4096}, int64_t{256}}) {
    const int64_t T = 16, S = 8192, RB = 512;
    std::vector<int64_t> slots(N);
    for (int64_t i = 0; i < N; i++) slots[i] = (i / 16) * 32 + (i % 16);  // runs of 16, gaps
    for (int64_t i = 0; i < N; i += 97) slots[i] = -1;
    std::vector<uint8_t> stage(T * N * RB);
    for (auto& b : stage) b = static_cast<uint8_t>(rng());
    std::vector<int64_t> offs(T);
    for (int64_t k = 0; k < T; k++) offs[k] = k * N * RB;
    std::vector<std::vector<uint8_t>> tab(T, std::vector<uint8_t>(S * RB));
    std::vector<std::vector<uint64_t>> ws(T, std::vector<uint64_t>(S));
    std::vector<std::vector<uint32_t>> crc(T, std::vector<uint32_t>(S));
    std::vector<void*> tp(T); std::vector<uint64_t*> wp(T); std::vector<uint32_t*> cp(T);
    for (int64_t k = 0; k < T; k++) { tp[k] = tab[k].data(); wp[k] = ws[k].data(); cp[k] = crc[k].data(); }
    int64_t fresh = -1;
    int rc = evs_store_commit(stage.data(), stage.size(), offs.data(), T, tp.data(), wp.data(),
                              cp.data(), S, RB, slots.data(), N, 5, 16, &fresh);
    CHECK(rc == 0);
    int64_t want_fresh = 0;
    for (int64_t k = 0; k < T; k++)
      for (int64_t i = 0; i < N; i++) {
        if (slots[i] < 0) continue;
        CHECK(std::memcmp(&tab[k][slots[i] * RB], &stage[offs[k] + i * RB], RB) == 0);
        CHECK(ws[k][slots[i]] == 5);
        uint32_t c; evs_crc32c(&tab[k][slots[i] * RB], RB, &c);
        CHECK(crc[k][slots[i]] == c);
      }
    for (int64_t i = 0; i < N; i++) want_fresh += slots[i] >= 0;
    CHECK(fresh == want_fresh * T);
    // a bad slot is refused before anything is written
    std::vector<int64_t> bad = slots; bad[N - 1] = S;
    CHECK(evs_store_commit(stage.data(), stage.size(), offs.data(), T, tp.data(), wp.data(),
                           cp.data(), S, RB, bad.data(), N, 6, 16, &fresh) != 0);
    CHECK(ws[0][slots[1]] == 5);
  }
  // host gather: 64 MiB of ranges on 8 threads
  const int64_t SR = 262144, RB2 = 256;
  std::vector<uint8_t> src(SR * RB2);
  for (auto& b : src) b = static_cast<uint8_t>(rng());
  std::vector<int64_t> st, ct;
  for (int64_t s = 0; s + 40 < SR; s += 41) { st.push_back(s); ct.push_back(1 + (s % 40)); }
  int64_t total = 0; for (auto c : ct) total += c;
  std::vector<uint8_t> dst(total * RB2);
  int64_t rows = 0;
  CHECK(evs_host_gather_ranges(src.data(), SR, RB2, st.data(), ct.data(), st.size(), dst.data(), total,
                               8, &rows) == 0);
  CHECK(rows == total);
  int64_t at = 0;
  for (size_t k = 0; k < st.size(); k++) {
    CHECK(std::memcmp(&dst[at * RB2], &src[st[k] * RB2], ct[k] * RB2) == 0);
    at += ct[k];
  }
  CHECK(evs_host_gather_ranges(src.data(), SR, RB2, st.data(), ct.data(), st.size(), dst.data(),
                               total - 1, 8, &rows) != 0);
  // several tables with the same ranges on 8 threads, each into its own block of dst
  const int64_t NT = 5;
  std::vector<std::vector<uint8_t>> srcs(NT, std::vector<uint8_t>(SR * RB2 / 8));
  std::vector<const void*> sp(NT);
  for (int64_t j = 0; j < NT; j++) {
    for (auto& b : srcs[j]) b = static_cast<uint8_t>(rng());
    sp[j] = srcs[j].data();
  }
  std::vector<int64_t> st2, ct2;
  for (int64_t s = 0; s + 40 < SR / 8; s += 53) { st2.push_back(s); ct2.push_back(1 + (s % 40)); }
  int64_t total2 = 0; for (auto c : ct2) total2 += c;
  const int64_t room = total2 + 3;
  std::vector<uint8_t> dst2(NT * room * RB2, 0xEE);
  CHECK(evs_host_gather_tables(sp.data(), NT, SR / 8, RB2, st2.data(), ct2.data(), st2.size(),
                               dst2.data(), room, 8, &rows) == 0);
  CHECK(rows == total2);
  for (int64_t j = 0; j < NT; j++) {
    int64_t at2 = 0;
    for (size_t k = 0; k < st2.size(); k++) {
      CHECK(std::memcmp(&dst2[(j * room + at2) * RB2], &srcs[j][st2[k] * RB2], ct2[k] * RB2) == 0);
      at2 += ct2[k];
    }
    for (int64_t b = total2 * RB2; b < room * RB2; b++) CHECK(dst2[j * room * RB2 + b] == 0xEE);
  }
  // two callers at once: one has the library's worker set, the other runs on threads of its own
  {
    std::vector<uint8_t> d1(NT * room * RB2, 0), d2(NT * room * RB2, 0);
    int64_t r1 = 0, r2 = 0;
    int rc1 = -1, rc2 = -1;
    for (int round = 0; round < 20; round++) {
      std::thread a([&] { rc1 = evs_host_gather_tables(sp.data(), NT, SR / 8, RB2, st2.data(),
                                                      ct2.data(), st2.size(), d1.data(), room, 8,
                                                      &r1); });
      std::thread b([&] { rc2 = evs_host_gather_tables(sp.data(), NT, SR / 8, RB2, st2.data(),
                                                      ct2.data(), st2.size(), d2.data(), room, 8,
                                                      &r2); });
      a.join();
      b.join();
      CHECK(rc1 == 0 && rc2 == 0 && r1 == total2 && r2 == total2);
    }
    for (int64_t j = 0; j < NT; j++)
      CHECK(std::memcmp(&d1[j * room * RB2], &dst2[j * room * RB2], total2 * RB2) == 0 &&
            std::memcmp(&d2[j * room * RB2], &dst2[j * room * RB2], total2 * RB2) == 0);
  }
  // crc rows: 4-row interleave and tails
  std::vector<uint32_t> out(1001);
  CHECK(evs_crc32c_rows(src.data(), 77, 1001, out.data()) == 0);
  for (int r = 0; r < 1001; r++) { uint32_t c; evs_crc32c(&src[r * 77], 77, &c); CHECK(out[r] == c); }
  std::printf("%s (%d failures)\n", fails ? "FAILED" : "ok", fails);
  return fails != 0;
}
