/*
 * oracle.c — a CPU restatement of the reference's per-worker KV data path. TEST INFRASTRUCTURE
 * ONLY: tests/, __graft_entry__.smoke() and bench.py's cpu_baseline leg use it as the checker.
 * The product (everserve_amd/) never links, loads or calls it.
 *
 * Scalar loops, one element at a time, written from the reference's definitions, not from the
 * HIP kernels. Built with gcc -O2 -ffp-contract=off (no fused or reassociated float arithmetic).
 */
#include <stdint.h>
#include <string.h>

/*
 * gather: core/csrc/gather.cu:29-47 (gather_elements) and core/everserve/state/kvcopy.py:89-116
 * (rows_of_heads, layout_strides), with the padding rule of gather.cu:37-38 and mirror.py:579:
 *
 *   out[l][h][t][k][j] = layer_l[(s / bs) * S0 + (s % bs) * S1 + heads[h] * S2 + k * S3 + j * S4],
 *   s = max(slots[t], 0), for l < L, h < H, t < n, k < 2, j < d; rows n..capacity-1 untouched.
 */
void orc_gather_rows(const void* const* layers, int64_t L, const int64_t* slots, int64_t n,
                     const int64_t* heads, int64_t H, void* out, int64_t capacity, int64_t d,
                     int64_t bs, const int64_t* S, int64_t elem) {
  unsigned char* o = (unsigned char*)out;
  for (int64_t l = 0; l < L; l++) {
    const unsigned char* src = (const unsigned char*)layers[l];
    for (int64_t h = 0; h < H; h++) {
      for (int64_t t = 0; t < n; t++) {
        int64_t s = slots[t] < 0 ? 0 : slots[t];
        for (int64_t k = 0; k < 2; k++) {
          for (int64_t j = 0; j < d; j++) {
            int64_t at = (s / bs) * S[0] + (s % bs) * S[1] + heads[h] * S[2] + k * S[3] + j * S[4];
            int64_t to = ((((l * H + h) * capacity + t) * 2 + k) * d + j);
            memcpy(o + to * elem, src + at * elem, (size_t)elem);
          }
        }
      }
    }
  }
}

/*
 * scatter: the inverse, core/everserve/state/kvcopy.py:118-128 (write_rows) as the restore uses
 * it (core/everserve/state/mirror.py:926-937): layer_l[...same index...] = rows[l][h][t][k][j]
 * for every t with slots[t] >= 0. A negative slot is padding: the store never holds it
 * (store/src/storage.rs:926-929), so nothing is written for it.
 */
void orc_scatter_rows(void* const* layers, int64_t L, const int64_t* slots, int64_t n,
                      const int64_t* heads, int64_t H, const void* rows, int64_t capacity,
                      int64_t d, int64_t bs, const int64_t* S, int64_t elem) {
  const unsigned char* in = (const unsigned char*)rows;
  for (int64_t l = 0; l < L; l++) {
    unsigned char* dst = (unsigned char*)layers[l];
    for (int64_t h = 0; h < H; h++) {
      for (int64_t t = 0; t < n; t++) {
        int64_t s = slots[t];
        if (s < 0) continue;
        for (int64_t k = 0; k < 2; k++) {
          for (int64_t j = 0; j < d; j++) {
            int64_t at = (s / bs) * S[0] + (s % bs) * S[1] + heads[h] * S[2] + k * S[3] + j * S[4];
            int64_t from = ((((l * H + h) * capacity + t) * 2 + k) * d + j);
            memcpy(dst + at * elem, in + from * elem, (size_t)elem);
          }
        }
      }
    }
  }
}

/*
 * scatter by pairs: for i = 0 .. n-1, in listed order, staged row rows_of[i] is written at slot
 * slots[i] exactly as orc_scatter_rows writes row t at slots[t]; a negative slot, or a row
 * outside [0, capacity), writes nothing. orc_scatter_rows is the case rows_of[i] = i. The
 * reference has no such call: it is its restore write (kvcopy.py:118-128) with the staged row of
 * each slot named, so that a caller can choose the order of the writes.
 */
void orc_scatter_pairs(void* const* layers, int64_t L, const int64_t* slots,
                       const int64_t* rows_of, int64_t n, const int64_t* heads, int64_t H,
                       const void* rows, int64_t capacity, int64_t d, int64_t bs, const int64_t* S,
                       int64_t elem) {
  const unsigned char* in = (const unsigned char*)rows;
  for (int64_t l = 0; l < L; l++) {
    unsigned char* dst = (unsigned char*)layers[l];
    for (int64_t h = 0; h < H; h++) {
      for (int64_t i = 0; i < n; i++) {
        int64_t s = slots[i], t = rows_of[i];
        if (s < 0 || t < 0 || t >= capacity) continue;
        for (int64_t k = 0; k < 2; k++) {
          for (int64_t j = 0; j < d; j++) {
            int64_t at = (s / bs) * S[0] + (s % bs) * S[1] + heads[h] * S[2] + k * S[3] + j * S[4];
            int64_t from = ((((l * H + h) * capacity + t) * 2 + k) * d + j);
            memcpy(dst + at * elem, in + from * elem, (size_t)elem);
          }
        }
      }
    }
  }
}

static float bf16_to_float(uint16_t b) {
  uint32_t u = (uint32_t)b << 16;
  float f;
  memcpy(&f, &u, 4);
  return f;
}

/*
 * float -> bfloat16 as torch's .to(torch.bfloat16) does it (c10 round_to_nearest_even): a NaN
 * of either sign becomes 0x7FC0; otherwise round to nearest, ties to even, on the bit pattern.
 */
uint16_t orc_float_to_bf16(float f) {
  uint32_t u;
  memcpy(&u, &f, 4);
  if ((u & 0x7fffffffu) > 0x7f800000u) return 0x7fc0u;
  uint32_t bias = 0x7fffu + ((u >> 16) & 1u);
  return (uint16_t)((u + bias) >> 16);
}

/*
 * member_sum: core/everserve/reference/arith/ops.py:63-73, the reference reduction the slot
 * kernel equals bit for bit (core/tests/test_slot_kernel.py:216-234): acc = 0.0f; acc +=
 * float(x_m) for each member in the given order; out = bf16(acc). A NULL member is one whose
 * payload never arrived and contributes +0.0f, as the kernel's aborted reads do
 * (core/csrc/slot.cu:148).
 */
void orc_member_sum_bf16(const uint16_t* const* inputs, int64_t k, uint16_t* out, int64_t n) {
  for (int64_t i = 0; i < n; i++) {
    float acc = 0.0f;
    for (int64_t m = 0; m < k; m++) acc += inputs[m] != 0 ? bf16_to_float(inputs[m][i]) : 0.0f;
    out[i] = orc_float_to_bf16(acc);
  }
}
