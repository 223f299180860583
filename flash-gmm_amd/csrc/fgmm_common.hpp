// Device-side helpers shared by the Flash-GMM E-step kernels (gfx950, wave64).
#pragma once

#include <hip/hip_runtime.h>
#include <stdint.h>

#include "flashgmm.h"

namespace fgmm {

typedef float f32x4 __attribute__((ext_vector_type(4)));
typedef float f32x16 __attribute__((ext_vector_type(16)));

constexpr double kLog2e = 1.4426950408889634;
constexpr double kLn2 = 0.6931471805599453;
constexpr double kLog2Pi = 1.8378770664093453;  // log(2*pi), flash_gmm.py:91

// One 32x32x2 fp32 matrix-core step: C += A(32x2) * B(2x32).
// Lane layout of v_mfma_f32_32x32x2f32 on a 64-wide wavefront:
//   A: lane l holds A[m = l % 32][k = l / 32]
//   B: lane l holds B[k = l / 32][n = l % 32]
//   C: lane l, accumulator register i holds C[m = acc_row(i, l / 32)][n = l % 32]
__device__ __forceinline__ f32x16 mfma32(float a, float b, f32x16 c) {
  return __builtin_amdgcn_mfma_f32_32x32x2f32(a, b, c, 0, 0, 0);
}

__host__ __device__ constexpr int acc_row(int i, int g) { return 8 * (i >> 2) + 4 * g + (i & 3); }

__device__ __forceinline__ f32x16 zero16() {
  f32x16 z;
#pragma unroll
  for (int i = 0; i < 16; ++i) z[i] = 0.0f;
  return z;
}

__device__ __forceinline__ f32x4 zero4() {
  f32x4 z = {0.0f, 0.0f, 0.0f, 0.0f};
  return z;
}

// 16-byte load of X[row][d0 .. d0+3] with the columns at or beyond D zeroed.
// The caller guarantees ldx >= round_up(D, 4), so the whole vector lies inside
// the row whenever d0 < D.
__device__ __forceinline__ f32x4 load_row4(const float* __restrict__ X, int64_t ldx, int64_t row,
                                           int d0, int D, bool valid) {
  f32x4 v = zero4();
  if (valid && d0 < D) {
    v = *reinterpret_cast<const f32x4*>(X + row * ldx + d0);
    if (d0 + 1 >= D) v.y = 0.0f;
    if (d0 + 2 >= D) v.z = 0.0f;
    if (d0 + 3 >= D) v.w = 0.0f;
  }
  return v;
}

__device__ __forceinline__ float fast_exp2(float x) { return __builtin_amdgcn_exp2f(x); }

// One 32x32 output tile of a D-contraction, sum_d A[m][d] B[d][n], returned in
// fp64 per accumulator register.  loadA(m) / loadB(m) give this lane's operand
// chunk m: four consecutive values of its dimension slice 8m + 4*(lane/32) .. +3.
// Each chunk of 8 dimensions is 4 fp32 MFMA steps from a zero accumulator; the
// chunk sums are then added in fp64, which bounds the fp32 rounding to one
// 8-term partial sum per chunk.
//
// Software pipeline: iteration m issues the MFMA chain of chunk m, adds chunk
// m-1 (whose chain has finished) into the fp64 sums, and loads the operands of
// chunk m+1.  The empty asm statements and the scheduling barrier keep the
// compiler from deferring the flushes, which would hold every chunk's
// accumulator live at once.
__device__ __forceinline__ f32x16 mfma_chunk(const f32x4 a, const f32x4 b) {
  f32x16 c = mfma32(a[0], b[0], zero16());
  c = mfma32(a[1], b[1], c);
  c = mfma32(a[2], b[2], c);
  return mfma32(a[3], b[3], c);
}

template <int NM, typename LA, typename LB>
__device__ __forceinline__ void cross_tile(double (&out)[16], LA loadA, LB loadB) {
  f32x4 a = loadA(0), b = loadB(0);
  f32x4 an = a, bn = b;
  if (NM > 1) {
    an = loadA(1);
    bn = loadB(1);
  }
  f32x16 prev = mfma_chunk(a, b);
#pragma unroll
  for (int m = 1; m < NM; ++m) {
    a = an;
    b = bn;
    if (m + 1 < NM) {
      an = loadA(m + 1);
      bn = loadB(m + 1);
    }
    const f32x16 cur = mfma_chunk(a, b);
    if (m == 1) {
#pragma unroll
      for (int i = 0; i < 16; ++i) out[i] = (double)prev[i];
    } else {
#pragma unroll
      for (int i = 0; i < 16; ++i) out[i] += (double)prev[i];
    }
    // Materialise the fp64 sums here: without this, IR-level sinking moves every
    // flush down to the first use of out[] and keeps all chunk results live.
#pragma unroll
    for (int i = 0; i < 16; ++i) asm volatile("" : "+v"(out[i]));
    prev = cur;
    __builtin_amdgcn_sched_barrier(0);
  }
  if (NM == 1) {
#pragma unroll
    for (int i = 0; i < 16; ++i) out[i] = (double)prev[i];
  } else {
#pragma unroll
    for (int i = 0; i < 16; ++i) out[i] += (double)prev[i];
  }
}

__host__ __device__ constexpr int64_t cdiv(int64_t a, int64_t b) { return (a + b - 1) / b; }
__host__ __device__ constexpr int64_t round_up(int64_t a, int64_t b) { return cdiv(a, b) * b; }

__host__ inline size_t align256(size_t x) { return (x + 255) & ~size_t(255); }

}  // namespace fgmm
