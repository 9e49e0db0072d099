// Philox4x64-10 counter-based generator (Salmon et al., "Parallel Random
// Numbers: As Easy as 1, 2, 3", SC'11). Multipliers and Weyl constants are
// the published Philox4x64 values. Usable from host and device code.
//
// Counter convention used across this library: word i of stream
// (key0, key1) is block (counter = i/4 + 1, 0, 0, 0) word i % 4, the same
// convention numpy.random.Philox uses (it increments the counter before each
// block), so numpy's random_raw() pins the implementation.
#pragma once
#include <cstdint>

#if defined(__HIPCC__)
#define SH_HD __host__ __device__ inline
#else
#define SH_HD static inline
#endif

SH_HD void sh_mulhilo64(uint64_t a, uint64_t b, uint64_t* hi, uint64_t* lo) {
  unsigned __int128 p = (unsigned __int128)a * (unsigned __int128)b;
  *hi = (uint64_t)(p >> 64);
  *lo = (uint64_t)p;
}

SH_HD void sh_philox4x64_10(const uint64_t ctr_in[4], const uint64_t key_in[2], uint64_t out[4]) {
  const uint64_t M0 = 0xD2E7470EE14C6C93ull, M1 = 0xCA5A826395121157ull;
  const uint64_t W0 = 0x9E3779B97F4A7C15ull, W1 = 0xBB67AE8584CAA73Bull;
  uint64_t c0 = ctr_in[0], c1 = ctr_in[1], c2 = ctr_in[2], c3 = ctr_in[3];
  uint64_t k0 = key_in[0], k1 = key_in[1];
  for (int r = 0; r < 10; ++r) {
    uint64_t hi0, lo0, hi1, lo1;
    sh_mulhilo64(M0, c0, &hi0, &lo0);
    sh_mulhilo64(M1, c2, &hi1, &lo1);
    uint64_t n0 = hi1 ^ c1 ^ k0;
    uint64_t n1 = lo1;
    uint64_t n2 = hi0 ^ c3 ^ k1;
    uint64_t n3 = lo0;
    c0 = n0; c1 = n1; c2 = n2; c3 = n3;
    k0 += W0;
    k1 += W1;
  }
  out[0] = c0; out[1] = c1; out[2] = c2; out[3] = c3;
}

// Uniform float in [0, 1) from one 64-bit word: top 24 bits * 2^-24 (exact).
SH_HD float sh_u64_to_unit_f32(uint64_t w) { return (float)(uint32_t)(w >> 40) * 0x1.0p-24f; }
