// Checks the SIMD Philox sweeps of the host row generator (AVX2 and AVX-512)
// against the scalar philox10() word for word.  Built and run by tests/test_rng.py
// with the generator's source included directly (its helpers have internal linkage).
#include "fgmm_rng_host.cpp"
#include <cstdio>
int main() {
  const int64_t m = 64;
  const bool avx512 = __builtin_cpu_supports("avx512f") && __builtin_cpu_supports("avx512bw") &&
                      __builtin_cpu_supports("avx512dq") && __builtin_cpu_supports("avx512vl");
  alignas(64) uint32_t a0[m], a1[m], a2[m], a3[m], b0[m], b1[m], b2[m], b3[m];
  for (int i = 0; i < m; ++i) { a0[i] = b0[i] = 0x12345678u * i + 7; a1[i] = b1[i] = i; a2[i] = b2[i] = 3 * i + 1; a3[i] = b3[i] = 0x6E6F6973u; }
  philox_sweep_avx2(a0, a1, a2, a3, m, 0xDEADBEEFu, 0x01234567u);
  if (avx512) philox_sweep_avx512(b0, b1, b2, b3, m, 0xDEADBEEFu, 0x01234567u);
  int bad = 0;
  for (int i = 0; i < m; ++i) {
    Ctr r = philox10(Ctr{{0x12345678u * i + 7, (uint32_t)i, 3u * i + 1, 0x6E6F6973u}}, 0xDEADBEEFu, 0x01234567u);
    bad += (r.v[0] != a0[i]) + (r.v[1] != a1[i]) + (r.v[2] != a2[i]) + (r.v[3] != a3[i]);
    if (avx512) bad += (r.v[0] != b0[i]) + (r.v[1] != b1[i]) + (r.v[2] != b2[i]) + (r.v[3] != b3[i]);
  }
  printf("mismatches: %d (avx512 %s)\n", bad, avx512 ? "checked" : "not available");
  return bad != 0;
}
