// Host-side synthetic row source for the streaming EM driver (plain C++, no HIP).
//
// Rows follow the clustered isotropic model: x_n = c[a_n] + z_n, a_n uniform over
// the K centres, z_n ~ N(0, I).  Randomness is counter-based: Philox4x32-10
// (Salmon, Moraes, Dror, Shaw, "Parallel random numbers: as easy as 1, 2, 3",
// SC'11) keyed by the seed, with the counter (row, block, 0, tag), so row n is the
// same whatever chunk or thread produces it.  Normals come from the Box-Muller
// transform of two 24-bit uniforms in (0, 1); the four normals of counter block j
// of a row are its coordinates j, J+j, 2J+j and 3J+j (J = D/4, rounded up; the
// ones at or beyond D are dropped).
#include <immintrin.h>
#include <stdint.h>
#include <stdlib.h>

#include <algorithm>
#include <math.h>
#include <memory>
#include <thread>
#include <vector>

#include "flashgmm.h"

namespace {

struct Ctr {
  uint32_t v[4];
};

inline void mulhilo(uint32_t a, uint32_t b, uint32_t& hi, uint32_t& lo) {
  const uint64_t p = (uint64_t)a * (uint64_t)b;
  hi = (uint32_t)(p >> 32);
  lo = (uint32_t)p;
}

// Ten Philox4x32 rounds: multipliers 0xD2511F53 / 0xCD9E8D57, Weyl key increments
// 0x9E3779B9 / 0xBB67AE85 (the published constants of the generator).
inline Ctr philox10(Ctr c, uint32_t k0, uint32_t k1) {
  for (int r = 0; r < 10; ++r) {
    uint32_t hi0, lo0, hi1, lo1;
    mulhilo(0xD2511F53u, c.v[0], hi0, lo0);
    mulhilo(0xCD9E8D57u, c.v[2], hi1, lo1);
    c = Ctr{{hi1 ^ c.v[1] ^ k0, lo1, hi0 ^ c.v[3] ^ k1, lo0}};
    k0 += 0x9E3779B9u;
    k1 += 0xBB67AE85u;
  }
  return c;
}

inline float u01(uint32_t x) { return ((float)(x >> 8) + 0.5f) * (1.0f / 16777216.0f); }

constexpr uint32_t kTagNoise = 0x6E6F6973u;   // counter word 3 for noise blocks
constexpr uint32_t kTagAssign = 0x61737367u;  // counter word 3 for the assignment draw

// Rows are produced in batches of kBatch, in vectorisable sweeps over the batch's
// counter blocks: Philox for every (row, block), the Box-Muller radius and angle,
// cos, sin, then the centre.  Per-block state lives in structure-of-arrays buffers
// so the compiler maps the 32x32->64 multiplies and the log / sqrt / sin / cos
// calls to SIMD code (glibc's vector math library).  Every sweep covers a whole
// number of 16-lane vectors over 64-byte aligned buffers, so no element takes a
// scalar prologue or epilogue and a row's value does not depend on where in a
// batch it falls.  The body is compiled twice, for AVX-512 and for AVX2
// (x86-64-v3), and fill_rows picks the one the host supports; values are
// reproducible for a given host instruction set.
constexpr int64_t kBatch = 16;

struct FreeDeleter {
  void operator()(void* p) const { free(p); }
};
template <typename T>
std::unique_ptr<T[], FreeDeleter> aligned_buffer(int64_t n) {
  const size_t bytes = ((size_t)n * sizeof(T) + 63) & ~size_t(63);
  return std::unique_ptr<T[], FreeDeleter>(static_cast<T*>(aligned_alloc(64, bytes)));
}

// Ten Philox rounds over m counter blocks held as four word arrays (m a multiple
// of 16, 64-byte aligned), 16 (AVX-512) or 8 (AVX2) blocks per vector.  The high
// half of each 32x32 product comes from two 32x32->64 multiplies (even and odd
// lanes) and a lane blend, the low half from a 32-bit multiply; results equal the
// scalar philox10() word for word.
__attribute__((target("avx512f,avx512bw,avx512dq,avx512vl")))
void philox_sweep_avx512(uint32_t* c0, uint32_t* c1, uint32_t* c2, uint32_t* c3, int64_t m,
                         uint32_t k0, uint32_t k1) {
  const __m512i M0 = _mm512_set1_epi32((int)0xD2511F53u), M1 = _mm512_set1_epi32((int)0xCD9E8D57u);
  for (int64_t i = 0; i < m; i += 16) {
    __m512i x0 = _mm512_load_si512(c0 + i), x1 = _mm512_load_si512(c1 + i);
    __m512i x2 = _mm512_load_si512(c2 + i), x3 = _mm512_load_si512(c3 + i);
    uint32_t a = k0, b = k1;
    for (int r = 0; r < 10; ++r) {
      const __m512i lo0 = _mm512_mullo_epi32(x0, M0), lo1 = _mm512_mullo_epi32(x2, M1);
      const __m512i hi0 = _mm512_mask_blend_epi32(
          0xAAAA, _mm512_srli_epi64(_mm512_mul_epu32(x0, M0), 32),
          _mm512_mul_epu32(_mm512_srli_epi64(x0, 32), M0));
      const __m512i hi1 = _mm512_mask_blend_epi32(
          0xAAAA, _mm512_srli_epi64(_mm512_mul_epu32(x2, M1), 32),
          _mm512_mul_epu32(_mm512_srli_epi64(x2, 32), M1));
      const __m512i n0 = _mm512_ternarylogic_epi32(hi1, x1, _mm512_set1_epi32((int)a), 0x96);
      const __m512i n2 = _mm512_ternarylogic_epi32(hi0, x3, _mm512_set1_epi32((int)b), 0x96);
      x1 = lo1;
      x3 = lo0;
      x0 = n0;
      x2 = n2;
      a += 0x9E3779B9u;
      b += 0xBB67AE85u;
    }
    _mm512_store_si512(c0 + i, x0);
    _mm512_store_si512(c1 + i, x1);
    _mm512_store_si512(c2 + i, x2);
    _mm512_store_si512(c3 + i, x3);
  }
}

void philox_sweep_avx2(uint32_t* c0, uint32_t* c1, uint32_t* c2, uint32_t* c3, int64_t m,
                       uint32_t k0, uint32_t k1) {
  const __m256i M0 = _mm256_set1_epi32((int)0xD2511F53u), M1 = _mm256_set1_epi32((int)0xCD9E8D57u);
  for (int64_t i = 0; i < m; i += 8) {
    __m256i x0 = _mm256_load_si256(reinterpret_cast<const __m256i*>(c0 + i));
    __m256i x1 = _mm256_load_si256(reinterpret_cast<const __m256i*>(c1 + i));
    __m256i x2 = _mm256_load_si256(reinterpret_cast<const __m256i*>(c2 + i));
    __m256i x3 = _mm256_load_si256(reinterpret_cast<const __m256i*>(c3 + i));
    uint32_t a = k0, b = k1;
    for (int r = 0; r < 10; ++r) {
      const __m256i lo0 = _mm256_mullo_epi32(x0, M0), lo1 = _mm256_mullo_epi32(x2, M1);
      const __m256i hi0 = _mm256_blend_epi32(_mm256_srli_epi64(_mm256_mul_epu32(x0, M0), 32),
                                             _mm256_mul_epu32(_mm256_srli_epi64(x0, 32), M0), 0xAA);
      const __m256i hi1 = _mm256_blend_epi32(_mm256_srli_epi64(_mm256_mul_epu32(x2, M1), 32),
                                             _mm256_mul_epu32(_mm256_srli_epi64(x2, 32), M1), 0xAA);
      const __m256i n0 = _mm256_xor_si256(_mm256_xor_si256(hi1, x1), _mm256_set1_epi32((int)a));
      const __m256i n2 = _mm256_xor_si256(_mm256_xor_si256(hi0, x3), _mm256_set1_epi32((int)b));
      x1 = lo1;
      x3 = lo0;
      x0 = n0;
      x2 = n2;
      a += 0x9E3779B9u;
      b += 0xBB67AE85u;
    }
    _mm256_store_si256(reinterpret_cast<__m256i*>(c0 + i), x0);
    _mm256_store_si256(reinterpret_cast<__m256i*>(c1 + i), x1);
    _mm256_store_si256(reinterpret_cast<__m256i*>(c2 + i), x2);
    _mm256_store_si256(reinterpret_cast<__m256i*>(c3 + i), x3);
  }
}

template <int ISA>
__attribute__((always_inline)) inline void fill_rows_body(const fgmm_synth_iso* s, int64_t row0,
                                                          int64_t nrows, float* dst) {
  const int64_t D = s->D;
  const int64_t J = (D + 3) / 4;
  const int64_t M = kBatch * J;
  const uint32_t k0 = (uint32_t)s->seed, k1 = (uint32_t)(s->seed >> 32);
  auto w0 = aligned_buffer<uint32_t>(M), w1 = aligned_buffer<uint32_t>(M);
  auto w2 = aligned_buffer<uint32_t>(M), w3 = aligned_buffer<uint32_t>(M);
  auto rad = aligned_buffer<float>(2 * M), ang = aligned_buffer<float>(2 * M);
  auto z = aligned_buffer<float>(4 * M);
  int64_t comp[kBatch];
  static_assert(kBatch % 16 == 0, "sweeps are multiples of the SIMD width");
  for (int64_t b0 = 0; b0 < nrows; b0 += kBatch) {
    const int64_t nb = std::min(kBatch, nrows - b0);
    uint32_t* c0 = w0.get();
    uint32_t* c1 = w1.get();
    uint32_t* c2 = w2.get();
    uint32_t* c3 = w3.get();
    // Full batches always: rows past nb get dummy counters and are discarded, so
    // every element takes the same (vector) code path and a row's value does not
    // depend on its position in a batch.
    for (int64_t b = 0; b < kBatch; ++b) {
      const uint64_t row = (uint64_t)(row0 + b0 + (b < nb ? b : 0));
      const uint32_t rlo = (uint32_t)row, rhi = (uint32_t)(row >> 32);
      const Ctr a = philox10(Ctr{{rlo, rhi, 0u, kTagAssign}}, k0, k1);
      comp[b] = (int64_t)(((uint64_t)a.v[0] * (uint64_t)s->K) >> 32);
      for (int64_t j = 0; j < J; ++j) {
        c0[b * J + j] = rlo;
        c1[b * J + j] = rhi;
        c2[b * J + j] = (uint32_t)j;
        c3[b * J + j] = kTagNoise;
      }
    }
    const int64_t m = M;
    if constexpr (ISA == 512)
      philox_sweep_avx512(c0, c1, c2, c3, m, k0, k1);
    else
      philox_sweep_avx2(c0, c1, c2, c3, m, k0, k1);
    // Box-Muller.  The radius/angle sweep comes first and sin and cos run in
    // separate sweeps: a fused sin/cos pair becomes a complex-exponential call
    // with no SIMD form.  Outputs: zA = r0 cos t0, zB = r0 sin t0, zC = r1 cos t1,
    // zD = r1 sin t1, each indexed by (row, block).
    float* ma = rad.get();
    float* mb = ma + M;
    float* ta = ang.get();
    float* tb = ta + M;
    float* zA = z.get();
    float* zB = zA + M;
    float* zC = zA + 2 * M;
    float* zD = zA + 3 * M;
    for (int64_t i = 0; i < m; ++i) {
      ma[i] = sqrtf(-2.0f * logf(u01(c0[i])));
      mb[i] = sqrtf(-2.0f * logf(u01(c2[i])));
      ta[i] = 6.283185307179586f * u01(c1[i]);
      tb[i] = 6.283185307179586f * u01(c3[i]);
    }
    for (int64_t i = 0; i < m; ++i) {
      zA[i] = ma[i] * cosf(ta[i]);
      zC[i] = mb[i] * cosf(tb[i]);
    }
    for (int64_t i = 0; i < m; ++i) {
      zB[i] = ma[i] * sinf(ta[i]);
      zD[i] = mb[i] * sinf(tb[i]);
    }
    // Coordinates of a row: block j's four normals are coordinates j, J+j, 2J+j, 3J+j.
    for (int64_t b = 0; b < nb; ++b) {
      const float* c = s->centres + comp[b] * D;
      float* out = dst + (b0 + b) * D;
      const float* q[4] = {zA + b * J, zB + b * J, zC + b * J, zD + b * J};
      for (int qd = 0; qd < 4; ++qd) {
        const int64_t d0 = qd * J;
        const int64_t len = std::min(J, D - d0);
        for (int64_t j = 0; j < len; ++j) out[d0 + j] = c[d0 + j] + q[qd][j];
      }
    }
  }
}

__attribute__((target("avx512f,avx512bw,avx512dq,avx512vl")))
void fill_rows_avx512(const fgmm_synth_iso* s, int64_t row0, int64_t nrows, float* dst) {
  fill_rows_body<512>(s, row0, nrows, dst);
}

void fill_rows_avx2(const fgmm_synth_iso* s, int64_t row0, int64_t nrows, float* dst) {
  fill_rows_body<256>(s, row0, nrows, dst);
}

void fill_rows(const fgmm_synth_iso* s, int64_t row0, int64_t nrows, float* dst) {
  static const bool avx512 = __builtin_cpu_supports("avx512f") && __builtin_cpu_supports("avx512bw") &&
                             __builtin_cpu_supports("avx512dq") && __builtin_cpu_supports("avx512vl");
  if (avx512)
    fill_rows_avx512(s, row0, nrows, dst);
  else
    fill_rows_avx2(s, row0, nrows, dst);
}

}  // namespace

extern "C" int fgmm_synth_iso_source(void* user, int64_t row0, int64_t nrows, int64_t D, float* dst) {
  const fgmm_synth_iso* s = static_cast<const fgmm_synth_iso*>(user);
  if (s == nullptr || dst == nullptr || s->centres == nullptr || D != s->D || s->K < 1 || row0 < 0 ||
      nrows < 0)
    return FGMM_ERR_INVALID_ARG;
  int T = s->threads > 0 ? s->threads : (int)std::max(1u, std::thread::hardware_concurrency());
  if ((int64_t)T > nrows) T = (int)std::max<int64_t>(1, nrows);
  if (T == 1) {
    fill_rows(s, row0, nrows, dst);
    return FGMM_OK;
  }
  std::vector<std::thread> pool;
  const int64_t per = (nrows + T - 1) / T;
  for (int t = 0; t < T; ++t) {
    const int64_t a = t * per, b = std::min(nrows, a + per);
    if (a >= b) break;
    pool.emplace_back(fill_rows, s, row0 + a, b - a, dst + a * D);
  }
  for (auto& th : pool) th.join();
  return FGMM_OK;
}
