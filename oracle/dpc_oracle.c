/*
 * C restatement of the integer/bit-level pieces of the device noise stream
 * (TEST INFRASTRUCTURE ONLY; compiled by oracle/build_oracle.py with gcc and
 * loaded by tests through ctypes).
 *
 * philox4x32_10: Salmon, Moraes, Dror, Shaw, "Parallel random numbers: as
 *   easy as 1, 2, 3" (SC'11), Philox4x32 with 10 rounds: multipliers
 *   0xD2511F53 / 0xCD9E8D57, key schedule increments 0x9E3779B9 / 0xBB67AE85.
 *   Pinned by the Random123 known-answer vectors (tests/test_oracle_noise.py).
 * normal_pair: the Box-Muller map of the device stream (53-bit radius
 *   uniform, 32-bit angle uniform) evaluated with the C library in double.
 */
#include <math.h>
#include <stddef.h>
#include <stdint.h>

void philox4x32_10(const uint32_t ctr[4], const uint32_t key[2], uint32_t out[4]) {
  uint32_t c0 = ctr[0], c1 = ctr[1], c2 = ctr[2], c3 = ctr[3];
  uint32_t k0 = key[0], k1 = key[1];
  for (int round = 0; round < 10; ++round) {
    uint64_t p0 = (uint64_t)0xD2511F53u * c0;
    uint64_t p1 = (uint64_t)0xCD9E8D57u * c2;
    uint32_t hi0 = (uint32_t)(p0 >> 32), lo0 = (uint32_t)p0;
    uint32_t hi1 = (uint32_t)(p1 >> 32), lo1 = (uint32_t)p1;
    uint32_t n0 = hi1 ^ c1 ^ k0;
    uint32_t n2 = hi0 ^ c3 ^ k1;
    c0 = n0;
    c1 = lo1;
    c2 = n2;
    c3 = lo0;
    k0 += 0x9E3779B9u;
    k1 += 0xBB67AE85u;
  }
  out[0] = c0;
  out[1] = c1;
  out[2] = c2;
  out[3] = c3;
}

void philox_many(uint32_t c0, uint32_t c1, uint32_t c2, uint32_t c3, uint32_t k0, uint32_t k1,
                 int n, uint32_t* out) {
  uint32_t key[2] = {k0, k1};
  for (int j = 0; j < n; ++j) {
    uint32_t ctr[4] = {c0 + (uint32_t)j, c1, c2, c3};
    philox4x32_10(ctr, key, out + 4 * (size_t)j);
  }
}

/* Standard-normal pair of Philox block `block` of leaf `leaf` under seed. */
void normal_pair(uint64_t seed, uint32_t leaf, uint64_t block, double* z0, double* z1) {
  uint32_t ctr[4] = {(uint32_t)block, (uint32_t)(block >> 32), leaf, 0u};
  uint32_t key[2] = {(uint32_t)seed, (uint32_t)(seed >> 32)};
  uint32_t w[4];
  philox4x32_10(ctr, key, w);
  uint64_t bits = ((uint64_t)w[0] << 32) | (uint64_t)w[1];
  double u1 = ((double)(bits >> 11) + 0.5) * 0x1.0p-53;
  double u2 = ((double)w[2] + 0.5) * 0x1.0p-32;
  double radius = sqrt(-2.0 * log(u1));
  double angle = 2.0 * M_PI * u2;
  *z0 = radius * cos(angle);
  *z1 = radius * sin(angle);
}

/* Normals for a leaf viewed as [rows, cols]: element (r, c) takes member
 * (r & 1) of block ((r >> 1) * cols + c). */
void leaf_normals(uint64_t seed, uint32_t leaf, int64_t rows, int64_t cols, double* out) {
  for (int64_t r = 0; r < rows; r += 2) {
    for (int64_t c = 0; c < cols; ++c) {
      double z0, z1;
      normal_pair(seed, leaf, (uint64_t)(r >> 1) * (uint64_t)cols + (uint64_t)c, &z0, &z1);
      out[r * cols + c] = z0;
      if (r + 1 < rows) out[(r + 1) * cols + c] = z1;
    }
  }
}
