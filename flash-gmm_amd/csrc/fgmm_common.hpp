// Device-side helpers shared by the Flash-GMM E-step kernels (gfx950, wave64).
#pragma once

#include <hip/hip_runtime.h>

#include <atomic>
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

// 16-byte load of X[row][d0 .. d0+3] with the columns at or beyond D zeroed (all
// four when !valid).  The caller guarantees ldx >= round_up(D, 4), ldx % 4 == 0 and
// d0 % 4 == 0, so the whole vector lies inside the row whenever d0 < D, and N >= 1.
// No branch: an unused lane loads from row 0 or dimension 0 instead (its address is
// selected, not skipped), so a sequence of these loads is issued back to back and
// stays in flight together; a branch per load would make each wait for its data
// before the next.
__device__ __forceinline__ f32x4 load_row4(const float* __restrict__ X, int64_t ldx, int64_t row,
                                           int d0, int D, bool valid) {
  const bool in = valid && d0 < D;
  const float* p = X + (valid ? row * ldx : (int64_t)0);
  const f32x4 v = *reinterpret_cast<const f32x4*>(p + (d0 < D ? d0 : 0));
  f32x4 r;
  r.x = in ? v.x : 0.0f;
  r.y = (in && d0 + 1 < D) ? v.y : 0.0f;
  r.z = (in && d0 + 2 < D) ? v.z : 0.0f;
  r.w = (in && d0 + 3 < D) ? v.w : 0.0f;
  return r;
}

__device__ __forceinline__ float fast_exp2(float x) { return __builtin_amdgcn_exp2f(x); }

// The fp32 matrix cores add the products of a 32x32x2 (or 16x16x4) step to the
// accumulator one at a time, rounding after each, so a single chain over D=128
// carries ~1e-4 absolute error in the cross term of clustered data; the log-joints
// are formed by the centred split-bf16 contraction below instead.  On gfx950 a
// matrix step leaves the SIMD's issue port free for part of its 32 cycles: VALU
// instructions of another wave (or later independent ones of the same wave) run
// there, about half of them hidden when two waves on a SIMD are in the same phase
// and nearly all when one runs its VALU work while the other runs matrix steps.

// ---------------------------------------------------------------------------
// bf16 matrix steps (the bf16 operand contracts of the reference's H100 kernels).
// v_mfma_f32_32x32x16_bf16: C(32x32) += A(32x16) * B(16x32), fp32 accumulation.
// Lane l holds A[m = l % 32][k = 8 (l / 32) + e] and B[k = 8 (l / 32) + e][n = l % 32]
// for e = 0..7; C is laid out as for the fp32 step (acc_row).
// ---------------------------------------------------------------------------
typedef __bf16 bf16x8 __attribute__((ext_vector_type(8)));

__device__ __forceinline__ f32x16 mfma_bf16(bf16x8 a, bf16x8 b, f32x16 c) {
  return __builtin_amdgcn_mfma_f32_32x32x16_bf16(a, b, c, 0, 0, 0);
}

// Round-to-nearest-even fp32 -> bf16 of 8 values.
__device__ __forceinline__ bf16x8 to_bf16x8(f32x4 lo, f32x4 hi) {
  bf16x8 v;
  v[0] = (__bf16)lo.x; v[1] = (__bf16)lo.y; v[2] = (__bf16)lo.z; v[3] = (__bf16)lo.w;
  v[4] = (__bf16)hi.x; v[5] = (__bf16)hi.y; v[6] = (__bf16)hi.z; v[7] = (__bf16)hi.w;
  return v;
}

// A tile in the accumulator layout (lane = column c, register i = row acc_row(i, g))
// rounded to bf16 and re-laid as the A operands of two 16-row steps: lane-half g of
// operand p gets rows 16p + 8g + e, e = 0..7.  Registers 4p'+j hold rows 8p' + 4g + j;
// packed to bf16 pairs, one swap across the half-waves per pair of dwords moves rows
// 8p' + 4(1-g) + j to the other half (e = 0..3 from the first pair, 4..7 from the
// second), with no trip through LDS.
// One of the two: registers 8p .. 8p + 7 of the tile, passed as r8[0 .. 7], form the
// operand of the 16-row step p.
__device__ __forceinline__ bf16x8 acc_to_row_operand(const float* r8) {
  typedef __bf16 bf16x2 __attribute__((ext_vector_type(2)));
  auto pack = [](float u, float v) {
    const bf16x2 t = {(__bf16)u, (__bf16)v};
    return *reinterpret_cast<const unsigned*>(&t);
  };
  uint4 wv;
#pragma unroll
  for (int hh = 0; hh < 2; ++hh) {
    const auto sw = __builtin_amdgcn_permlane32_swap(pack(r8[2 * hh], r8[2 * hh + 1]),
                                                     pack(r8[4 + 2 * hh], r8[5 + 2 * hh]), false, false);
    if (hh == 0) { wv.x = sw[0]; wv.z = sw[1]; } else { wv.y = sw[0]; wv.w = sw[1]; }
  }
  return *reinterpret_cast<const bf16x8*>(&wv);
}
__device__ __forceinline__ void acc_to_row_operands(const float (&r)[16], bf16x8 (&a)[2]) {
  a[0] = acc_to_row_operand(r);
  a[1] = acc_to_row_operand(r + 8);
}

// ---------------------------------------------------------------------------
// fp32 dot products on the bf16 matrix cores ("bf16x6", split-bf16 emulation).
// Each fp32 operand is split exactly into three bf16 values, v = v1 + v2 + v3
// (v1 = bf16(v), v2 = bf16(v - v1), v3 = bf16(v - v1 - v2); both differences are
// exact in fp32), and x.mu is formed from the six products of significance at
// least 2^-16: x2 mu2, x1 mu3, x3 mu1, x2 mu1, x1 mu2, x1 mu1 (the dropped ones are
// ~2^-24 of |x||mu|).  Measured on gfx950, v_mfma_f32_32x32x16_bf16 adds the 8
// products of each lane-half exactly after aligning them to the largest one (bits
// below 2^-24 of it are truncated), and rounds to nearest once per lane-half when
// adding to the accumulator.  Issuing the five small terms first into a zero
// accumulator and x1 mu1 last keeps the accumulator small until the final step,
// so a 16-dimension chunk carries about two fp32 roundings at its own magnitude.
// Six bf16 steps (192 matrix cycles) replace 8 fp32 steps (512 cycles) per 16
// dimensions.
// ---------------------------------------------------------------------------
// Two values at a time: one packed round-to-nearest-even conversion per pair
// (v_cvt_pk_bf16_f32), the bf16 halves widened back by a shift or a mask.
typedef float f32x2 __attribute__((ext_vector_type(2)));
typedef __bf16 bf16x2 __attribute__((ext_vector_type(2)));
__device__ __forceinline__ unsigned bf16_pair(f32x2 v) {
  return __builtin_bit_cast(unsigned, __builtin_convertvector(v, bf16x2));
}
__device__ __forceinline__ f32x2 bf16_pair_widen(unsigned w) {
  const f32x2 r = {__uint_as_float(w << 16), __uint_as_float(w & 0xffff0000u)};
  return r;
}

// acc_to_row_operand of registers already packed in bf16 pairs (w[j] = registers
// 2j, 2j + 1 of the eight).
__device__ __forceinline__ bf16x8 pairs_to_row_operand(const unsigned (&w)[4]) {
  uint4 wv;
#pragma unroll
  for (int hh = 0; hh < 2; ++hh) {
    const auto sw = __builtin_amdgcn_permlane32_swap(w[hh], w[2 + hh], false, false);
    if (hh == 0) { wv.x = sw[0]; wv.z = sw[1]; } else { wv.y = sw[0]; wv.w = sw[1]; }
  }
  return __builtin_bit_cast(bf16x8, wv);
}

// acc_to_row_operand of r8 (hi) and of its exact residuals r8 - bf16(r8) (lo): each
// pair is rounded once, and the residuals come from the widened rounding.
__device__ __forceinline__ void acc_to_row_operands_split(const float* r8, bf16x8& hi, bf16x8& lo) {
  unsigned ph[4], pl[4];
#pragma unroll
  for (int j = 0; j < 4; ++j) {
    const f32x2 v = {r8[2 * j], r8[2 * j + 1]};
    ph[j] = bf16_pair(v);
    pl[j] = bf16_pair(v - bf16_pair_widen(ph[j]));
  }
  hi = pairs_to_row_operand(ph);
  lo = pairs_to_row_operand(pl);
}

// The same with three parts: r8 = r1 + r2 + r3 exactly before r3's rounding
// (split3_bf16's parts, in the row-operand layout).
__device__ __forceinline__ void acc_to_row_operands_split3(const float* r8, bf16x8& a1, bf16x8& a2, bf16x8& a3) {
  unsigned p1[4], p2[4], p3[4];
#pragma unroll
  for (int j = 0; j < 4; ++j) {
    const f32x2 v = {r8[2 * j], r8[2 * j + 1]};
    p1[j] = bf16_pair(v);
    const f32x2 d1 = v - bf16_pair_widen(p1[j]);
    p2[j] = bf16_pair(d1);
    p3[j] = bf16_pair(d1 - bf16_pair_widen(p2[j]));
  }
  a1 = pairs_to_row_operand(p1);
  a2 = pairs_to_row_operand(p2);
  a3 = pairs_to_row_operand(p3);
}

__device__ __forceinline__ void split3_bf16(const f32x4 lo, const f32x4 hi, bf16x8 (&s)[3]) {
  const float v[8] = {lo.x, lo.y, lo.z, lo.w, hi.x, hi.y, hi.z, hi.w};
  uint4 w[3];
#pragma unroll
  for (int j = 0; j < 4; ++j) {
    const f32x2 a = {v[2 * j], v[2 * j + 1]};
    const unsigned h = bf16_pair(a);
    const f32x2 r = a - bf16_pair_widen(h);
    const unsigned m = bf16_pair(r);
    const unsigned l = bf16_pair(r - bf16_pair_widen(m));
    (j == 0 ? w[0].x : j == 1 ? w[0].y : j == 2 ? w[0].z : w[0].w) = h;
    (j == 0 ? w[1].x : j == 1 ? w[1].y : j == 2 ? w[1].z : w[1].w) = m;
    (j == 0 ? w[2].x : j == 1 ? w[2].y : j == 2 ? w[2].z : w[2].w) = l;
  }
#pragma unroll
  for (int t = 0; t < 3; ++t) s[t] = __builtin_bit_cast(bf16x8, w[t]);
}

// One 32x32 tile of the centred cross term t = x.mu - sum_q o_q over NQ
// 16-dimension chunks, where o_q is the fp32 value of ||mu_chunk q||^2 (the caller
// adds sum_q o_q back in fp64).  Per chunk: the five small terms, then -o_q (three
// bf16 values in k slots 0..2 of split 3 of the A operand, times the ones operand),
// then x1 mu1: for the components near a row the accumulator then stays small,
// and chunk q accumulates in chain q % MAXCH (independent chains cover the matrix
// latency; four by default), the chains being added in fp32 at the end.  The same
// form serves other feature layouts whose o_q centres the chunk (the diagonal
// model's [x^2, x] chunks).  loadA(q, s) returns split s
// of A-operand chunk q (lane: row m = lane % 32, dimensions 16q + 8(lane/32) + e),
// xb[q][s] the B operand.  CPU emulation of the hardware rules on the N=1M, K=1024,
// D=128 clustered data: max logZ error 4.5e-5 over 65,536 rows (4.2e-5 with the
// chunks summed in fp64, 5.5e-5 for fp32 steps on 8-dimension chunks).
template <int NQ, int MAXCH = 4, typename LA>
__device__ __forceinline__ f32x16 x6c_tile(LA loadA, const bf16x8 (&xb)[NQ][3], const bf16x8 ones) {
  constexpr int NCH = NQ < MAXCH ? NQ : MAXCH;
  f32x16 acc[NCH];
#pragma unroll
  for (int h = 0; h < NCH; ++h) acc[h] = zero16();
#pragma unroll
  for (int q0 = 0; q0 < NQ; q0 += NCH) {
    bf16x8 a[NCH][4];
#pragma unroll
    for (int h = 0; h < NCH; ++h) {
      if (q0 + h < NQ) {
#pragma unroll
        for (int t = 0; t < 4; ++t) a[h][t] = loadA(q0 + h, t);
      }
    }
    // Steps in order: x2 mu2, x1 mu3, x3 mu1, x2 mu1, x1 mu2, -o, x1 mu1.  A chunk's
    // seven steps are issued back to back (chain-major): consecutive matrix steps on
    // one accumulator use the hardware's accumulator forwarding, while alternating
    // two accumulators step by step measured 16% slower per step on gfx950.  The
    // order of the steps within each chain, and so every bit, is the same.
#pragma unroll
    for (int h = 0; h < NCH; ++h) {
      const int q = q0 + h;
      if (q < NQ) {
#pragma unroll
        for (int step = 0; step < 7; ++step) {
          const bf16x8 A = step == 0 ? a[h][1] : step == 1 ? a[h][2] : step <= 3 ? a[h][0]
                         : step == 4 ? a[h][1] : step == 5 ? a[h][3] : a[h][0];
          const bf16x8 B = step == 0 ? xb[q][1] : step == 1 ? xb[q][0] : step == 2 ? xb[q][2]
                         : step == 3 ? xb[q][1] : step == 4 ? xb[q][0] : step == 5 ? ones : xb[q][0];
          acc[h] = mfma_bf16(A, B, acc[h]);
        }
      }
    }
  }
  f32x16 t = acc[0];
#pragma unroll
  for (int h = 1; h < NCH; ++h) {
#pragma unroll
    for (int i = 0; i < 16; ++i) t[i] += acc[h][i];
  }
  return t;
}

// x6c_tile<NQ, 1> for T tiles of rows at once (xb[u] the B operand of tile u): each
// A operand read serves all T tiles, and every tile's steps, their order and its one
// chain are x6c_tile<NQ, 1>'s, so out[u] is the same bits as that call gives.
template <int NQ, int T, typename LA>
__device__ __forceinline__ void x6c_tile_multi(LA loadA, const bf16x8 (&xb)[T][NQ][3], const bf16x8 ones,
                                               f32x16 (&out)[T]) {
#pragma unroll
  for (int u = 0; u < T; ++u) out[u] = zero16();
#pragma unroll
  for (int q = 0; q < NQ; ++q) {
    bf16x8 a[4];
#pragma unroll
    for (int t = 0; t < 4; ++t) a[t] = loadA(q, t);
#pragma unroll
    for (int u = 0; u < T; ++u) {
#pragma unroll
      for (int step = 0; step < 7; ++step) {
        const bf16x8 A = step == 0 ? a[1] : step == 1 ? a[2] : step <= 3 ? a[0]
                       : step == 4 ? a[1] : step == 5 ? a[3] : a[0];
        const bf16x8 B = step == 0 ? xb[u][q][1] : step == 1 ? xb[u][q][0] : step == 2 ? xb[u][q][2]
                       : step == 3 ? xb[u][q][1] : step == 4 ? xb[u][q][0] : step == 5 ? ones : xb[u][q][0];
        out[u] = mfma_bf16(A, B, out[u]);
      }
    }
  }
}

// x6c_tile with the operand roles exchanged: A holds the rows' splits (lane m = row,
// xa[q][s] = split s of dimensions 16q + 8(lane/32) + e) and the ones operand of the
// offset step, B holds mu's splits and centring offsets (loadB(q, t), lane n =
// component).  The accumulator then holds C[row][component]: lane = component,
// register i = row acc_row(i, lane / 32), the layout whose rows feed r^T X.  The
// products, their order and the chains are x6c_tile's, and a matrix step's per-half
// sums do not depend on which operand is A, so every element equals the one
// x6c_tile forms for the same row and component.
template <int NQ, int MAXCH = 4, typename LB>
__device__ __forceinline__ f32x16 x6c_tile_rows(const bf16x8 (&xa)[NQ][3], const bf16x8 ones, LB loadB) {
  constexpr int NCH = NQ < MAXCH ? NQ : MAXCH;
  f32x16 acc[NCH];
#pragma unroll
  for (int h = 0; h < NCH; ++h) acc[h] = zero16();
#pragma unroll
  for (int q0 = 0; q0 < NQ; q0 += NCH) {
    bf16x8 b[NCH][4];
#pragma unroll
    for (int h = 0; h < NCH; ++h) {
      if (q0 + h < NQ) {
#pragma unroll
        for (int t = 0; t < 4; ++t) b[h][t] = loadB(q0 + h, t);
      }
    }
    // Chain-major, as x6c_tile.
#pragma unroll
    for (int h = 0; h < NCH; ++h) {
      const int q = q0 + h;
      if (q < NQ) {
#pragma unroll
        for (int step = 0; step < 7; ++step) {
          const bf16x8 B = step == 0 ? b[h][1] : step == 1 ? b[h][2] : step <= 3 ? b[h][0]
                         : step == 4 ? b[h][1] : step == 5 ? b[h][3] : b[h][0];
          const bf16x8 A = step == 0 ? xa[q][1] : step == 1 ? xa[q][0] : step == 2 ? xa[q][2]
                         : step == 3 ? xa[q][1] : step == 4 ? xa[q][0] : step == 5 ? ones : xa[q][0];
          acc[h] = mfma_bf16(A, B, acc[h]);
        }
      }
    }
  }
  f32x16 t = acc[0];
#pragma unroll
  for (int h = 1; h < NCH; ++h) {
#pragma unroll
    for (int i = 0; i < 16; ++i) t[i] += acc[h][i];
  }
  return t;
}

// B operand of a 16-row matrix step read from a row-major bf16 tile in LDS (row
// stride rs elements): lane l receives rows r0 + 8(l/32) + e, e = 0..7, of column
// c0 + l % 32.  ds_read_b64_tr_b16 (gfx950), measured: within each group of 16
// lanes, lane 4e + a supplies the address of 4 consecutive elements of one row,
// and lane 4a' + b' receives element b' of the rows supplied by lanes a', 4 + a',
// 8 + a' and 12 + a'.  Two reads (rows 8g .. 8g + 3, then 8g + 4 .. 8g + 7) give
// the operand.  A row stride of an odd multiple of 32 bytes keeps the 8 rows a
// read touches at most two to a bank.
typedef short i16x4 __attribute__((ext_vector_type(4)));
typedef __attribute__((address_space(3))) i16x4 lds_i16x4;

__device__ __forceinline__ bf16x8 lds_rows_operand(const __bf16* tile, int rs, int r0, int c0, int lane) {
  const int G = lane >> 4, i = lane & 15;
  const int row = r0 + 8 * (G >> 1) + (i >> 2);
  const int col = c0 + 16 * (G & 1) + 4 * (i & 3);
  const i16x4 lo = __builtin_amdgcn_ds_read_tr16_b64_v4i16((lds_i16x4*)(tile + row * rs + col));
  const i16x4 hi = __builtin_amdgcn_ds_read_tr16_b64_v4i16((lds_i16x4*)(tile + (row + 4) * rs + col));
  typedef short i16x8 __attribute__((ext_vector_type(8)));
  const i16x8 v = {lo[0], lo[1], lo[2], lo[3], hi[0], hi[1], hi[2], hi[3]};
  return __builtin_bit_cast(bf16x8, v);
}

// bf16 bit patterns rounded toward +infinity (a value never decreases), for
// upper bounds kept in half the space: truncation for negative values, round-up
// of the magnitude for positive ones; NaN stays NaN.
__device__ __forceinline__ unsigned short bf16_bits_up(float x) {
  // Selects, not branches (callers keep their loop bodies one scheduling region).
  const unsigned u = __float_as_uint(x);
  const unsigned up = (u & 0x80000000u) ? u : u + 0xffffu;
  return (unsigned short)(((u & 0x7fffffffu) > 0x7f800000u) ? 0x7fc0u : (up >> 16));
}
__device__ __forceinline__ float bf16_bits_to_float(unsigned short h) { return __uint_as_float((unsigned)h << 16); }

// The B operand of the offset step: 1 in k slots 0..2 (lane-half 0, elements 0..2).
__device__ __forceinline__ bf16x8 x6c_ones(int lane) {
  bf16x8 v;
#pragma unroll
  for (int e = 0; e < 8; ++e) v[e] = (__bf16)((lane < 32 && e < 3) ? 1.0f : 0.0f);
  return v;
}

// True when any lane's operand holds a nonzero bf16 (wave-uniform).
__device__ __forceinline__ bool any_nonzero(const bf16x8& a) {
  const uint4 bits = *reinterpret_cast<const uint4*>(&a);
  return __builtin_amdgcn_ballot_w64((bits.x | bits.y | bits.z | bits.w) != 0u) != 0;
}

// Sum of n floats p[0], p[stride], ... in fp64, left to right (a fixed order, so
// the result is deterministic); eight loads are issued before their adds.
__device__ __forceinline__ double strided_sum(const float* __restrict__ p, int n, int64_t stride) {
  double s = 0.0;
  int i = 0;
  for (; i + 8 <= n; i += 8) {
    float v[8];
#pragma unroll
    for (int u = 0; u < 8; ++u) v[u] = p[(int64_t)(i + u) * stride];
#pragma unroll
    for (int u = 0; u < 8; ++u) s += (double)v[u];
  }
  for (; i < n; ++i) s += (double)p[(int64_t)i * stride];
  return s;
}

// The same sum spread over the 64 lanes of a wave (for large n): lane l adds
// p[l], p[l + 64], ... in order, then a fixed xor butterfly combines the lanes.
// Deterministic; every lane returns the total.
__device__ __forceinline__ double wave_strided_sum(const float* __restrict__ p, int n, int64_t stride,
                                                   int lane) {
  double s = 0.0;
  for (int i = lane; i < n; i += 64) s += (double)p[(int64_t)i * stride];
#pragma unroll
  for (int o = 32; o >= 1; o >>= 1) s += __shfl_xor(s, o);
  return s;
}

// ---------------------------------------------------------------------------
// Stored log-joint.  Pass 1 can keep the fp32 log-joint (log2 units) of every
// (32-row tile, 32-component block) pair in the workspace, so that pass 2 reads
// it instead of recomputing the contraction.  Tiles are ordered (row tile,
// component block), 1024 floats each.  In the dense form below (diagonal
// covariances) they are in pass 1's register order: the pass-1
// lane l (row l % 32; component acc_row(i, l / 32) in register i) writes
// register i at i * 64 + l, so each store instruction fills 256 contiguous
// bytes.  Component k of row r therefore sits at
//     (4 * (k >> 3) + (k & 3)) * 64 + 32 * ((k >> 2) & 1) + r,
// and the pass-2 lane (component k = lane % 32, g = lane / 32), whose register
// i = 4q + j holds row 8q + 4g + j, reads four float4 at that offset for
// r = 8q + 4g.  The 4 loads of a wave cover each 128-byte line of the tile.
// ---------------------------------------------------------------------------
constexpr int kLjTile = 1024;   // floats per (row tile, component block)

// Workgroup barrier for LDS hand-offs.  __syncthreads() also drains every
// outstanding global access of the wave (vmcnt(0) on gfx9), which would stall on
// the log-joint stores and on loads prefetched for the next iteration; this one
// waits for the wave's LDS accesses only.  The memory clobber keeps the compiler
// from moving memory accesses across it.
__device__ __forceinline__ void lds_barrier() {
  asm volatile("s_waitcnt lgkmcnt(0)\n\ts_barrier" ::: "memory");
}

__device__ __forceinline__ void lj_store(float* __restrict__ tile, int lane, const double (&ll)[16]) {
#pragma unroll
  for (int i = 0; i < 16; ++i) __builtin_nontemporal_store((float)ll[i], tile + i * 64 + lane);
}

__device__ __forceinline__ void lj_load(const float* __restrict__ tile, int lane, f32x4 (&v)[4]) {
  const int k = lane & 31, g = lane >> 5;
  const float* p = tile + (4 * (k >> 3) + (k & 3)) * 64 + 32 * ((k >> 2) & 1) + 4 * g;
#pragma unroll
  for (int q = 0; q < 4; ++q) v[q] = *reinterpret_cast<const f32x4*>(p + 8 * q);
}

// ---------------------------------------------------------------------------
// Sparse stored log-joint (row-major tiles with need masks).
//
// On clustered data nearly every (row, component block) pair has a log-joint
// thousands of log2 units below the row's logZ2, so its responsibilities are
// exactly zero in fp32.  In this form a tile is stored row-major, tile[row * 32 +
// comp], so that one row of one block is one 128-byte line, and pass 1 leaves
// beside the tiles:
//   bmax[(tile, block)][row]  fp32 max of the row's 32 stored values;
//   mask[(tile, block)]       bit r set when row r may have a nonzero
//                             responsibility in the block.
// Pass 1 computes the masks after the row's logZ2 is final: with z = (hi, lo) the
// float pair pass 2 forms from logZ2, bit r is clear when
//     fl(fl(bmax - z.hi) - z.lo) < -kLjNeedGap.
// Rounding is monotone, so every value l <= bmax of the row then gives
// fl(fl(l - z.hi) - z.lo) < -kLjNeedGap as well.  Below -150, 2^x is under half
// the smallest fp32 denormal and v_exp_f32 returns 0, so the responsibilities pass
// 2 would form are exactly zero.  Pass 2 reads only the rows whose bit is set, so
// skipping the others changes no output bit.
//
// Pass 1 also leaves out the store of a row's block when the running max M of the
// row's stored values already proves the mask bit will be clear:
// fl(bmax - M) < -kLjSkipGap with |M| < 2^24.  logZ2 >= max log-joint >= M - 1
// (M is a float rounding of a log-joint), so bmax - logZ2 < 1 - kLjSkipGap, and the
// float evaluation above cannot reach -kLjNeedGap.  A half-wave whose block sum is
// NaN always stores (the row's logZ2 is NaN, so its mask bit is set).
// ---------------------------------------------------------------------------
constexpr float kLjNeedGap = 160.0f;
constexpr float kLjSkipGap = 192.0f;

// Max over both half-waves of the row's block maximum (lane = row in pass 1).
__device__ __forceinline__ float lj_row_max(double bm) {
  const unsigned u = __float_as_uint((float)bm);
  const auto s = __builtin_amdgcn_permlane32_swap(u, u, false, false);
  return fmaxf(__uint_as_float(s[0]), __uint_as_float(s[1]));
}

// Pass-1 store of one (row tile, block) pair, or of the part of it one wave holds.
// Lane (row c, half g) holds components acc_row(i, g), i.e. 8j + 4g + 0..3 in
// registers 4j..4j+3: NG float4 per lane for the register groups j0 .. j0 + NG - 1,
// the two halves together filling each row's line.  Each instruction writes 32 bytes
// of every row, so these are ordinary (write-back) stores that the L2 merges into
// whole lines; non-temporal ones reach HBM piecewise, at about twice the bytes.
// `bm` is the lane's max over its values, `lse_sum` the half-wave's running
// log-sum-exp sum after the block (NaN if any value was NaN), `run_max` the row's
// running max of the stored values it covers (updated here); `bmax` receives the max
// over both lane-halves.
template <int NG>
__device__ __forceinline__ void lj_put_rows_g(float* __restrict__ tile, float* __restrict__ bmax, int c,
                                              int g, int j0, const double (&ll)[4 * NG], double bm,
                                              float lse_sum, float& run_max, bool dense) {
  const float R = lj_row_max(bm);
  run_max = fmaxf(run_max, R);
  const bool skip = !dense && lse_sum == lse_sum && fabsf(run_max) < 0x1p24f && (R - run_max) < -kLjSkipGap;
  if (!skip) {
    float* p = tile + c * 32 + 4 * g;
#pragma unroll
    for (int j = 0; j < NG; ++j) {
      const f32x4 v = {(float)ll[4 * j], (float)ll[4 * j + 1], (float)ll[4 * j + 2], (float)ll[4 * j + 3]};
      *reinterpret_cast<f32x4*>(p + 8 * (j0 + j)) = v;
    }
  }
  if (g == 0) bmax[c] = R;
}

__device__ __forceinline__ void lj_put_rows(float* __restrict__ tile, float* __restrict__ bmax, int c,
                                            int g, const double (&ll)[16], double bm, float lse_sum,
                                            float& run_max, bool dense) {
  lj_put_rows_g<4>(tile, bmax, c, g, 0, ll, bm, lse_sum, run_max, dense);
}

// Pass-1 epilogue: need masks of the wave's row tile for all KB blocks.  Run by
// the half-wave g = 0 only (lane c = row c); each lane reads back the maxima it
// stored itself.  lz2 is the row's final logZ2; rows past N get no bit.  With
// `dense` (FGMM_FLAG_DENSE: every row stored) every row of the tile is marked, so a
// dense pass 2 reads and exponentiates all of them; pass 2 itself always follows
// the masks, whichever flags its own call carries.
//
// `count` gathers the number of register-row pairs (rows r and r + 4, r & 4 == 0:
// the two rows of one accumulation step) with a bit set, over the tile's blocks; the
// accumulation pass picks its sparse or dense form from the total.  The caller
// spreads tiles over 64 counters (one atomic per wave) that the prologue zeroes.
__device__ __forceinline__ unsigned lj_pair_mask(unsigned m) { return (m | (m >> 4)) & 0x0f0f0f0fu; }

// Block kb's maxima are at bmax[kb * bstride + c] and its mask at mask[kb * mstride]
// (strides 32 and 1 when one wave covers the whole block).
__device__ __forceinline__ void lj_put_masks(const float* __restrict__ bmax, unsigned* __restrict__ mask,
                                             unsigned* __restrict__ count, int KB, int c, double lz2,
                                             bool valid, bool dense, int bstride = 32, int mstride = 1) {
  const float zx = (float)lz2;
  const float zy = (lz2 > -INFINITY && lz2 < INFINITY) ? (float)(lz2 - (double)zx) : 0.0f;
  unsigned pairs = 0;
  for (int kb0 = 0; kb0 < KB; kb0 += 8) {
    float R[8];
#pragma unroll
    for (int j = 0; j < 8; ++j) R[j] = kb0 + j < KB ? bmax[(kb0 + j) * bstride + c] : 0.0f;
#pragma unroll
    for (int j = 0; j < 8; ++j) {
      if (kb0 + j < KB) {
        const bool need = valid && (dense || !(((R[j] - zx) - zy) < -kLjNeedGap));
        const unsigned b = (unsigned)__builtin_amdgcn_ballot_w64(need);
        pairs += __builtin_popcount(lj_pair_mask(b));
        if (c == 0) mask[(kb0 + j) * mstride] = b;
      }
    }
  }
  if (c == 0 && pairs != 0) atomicAdd(count, pairs);
}

// ---------------------------------------------------------------------------
// Need masks without a stored log-joint (the default, O(N + K*D) plan).  Pass 1
// keeps each row's block maximum R as a bf16 upper bound (bf16_bits_up) in LDS, one
// per (wave, block, row), and after the row's logZ2 is final sets bit r of the
// (tile, block) word unless fl(fl(R - z.hi) - z.lo) < -kLjNeedGap, the test above.
// R bounds every log-joint value the accumulation pass recomputes for the row and
// block (the same arithmetic), so a clear bit again means responsibilities that are
// exactly zero in fp32.  `rmax(kb)` returns the lane's bound for block kb.  Run by
// the half-wave g = 0 (lane c = row c); `count` gathers the number of bits set
// (needed (row, block) pairs), from which the accumulation pass picks its form.
template <typename RM>
__device__ __forceinline__ void need_put_masks(RM rmax, unsigned* __restrict__ mask, unsigned* __restrict__ count,
                                               int KB, int c, double lz2, bool valid, bool dense,
                                               int mstride = 1) {
  const float zx = (float)lz2;
  const float zy = (lz2 > -INFINITY && lz2 < INFINITY) ? (float)(lz2 - (double)zx) : 0.0f;
  unsigned pairs = 0;
  for (int kb0 = 0; kb0 < KB; kb0 += 8) {
    // Eight bounds in flight together: the index is clamped rather than the read
    // skipped, which would put a branch (and a wait) around each one.
    float R[8];
#pragma unroll
    for (int j = 0; j < 8; ++j) R[j] = rmax(kb0 + j < KB ? kb0 + j : KB - 1);
#pragma unroll
    for (int j = 0; j < 8; ++j) {
      if (kb0 + j < KB) {
        const bool need = valid && (dense || !(((R[j] - zx) - zy) < -kLjNeedGap));
        const unsigned b = (unsigned)__builtin_amdgcn_ballot_w64(need);
        pairs += __builtin_popcount(b);
        if (c == 0) mask[(kb0 + j) * mstride] = b;
      }
    }
  }
  if (count && c == 0 && pairs != 0) atomicAdd(count, pairs);
}

// Total of the 64 needed-pair counters pass 1 adds to, in 64 bits (needed rows of a
// call can pass 2^32); one wave, uniform result.
__device__ __forceinline__ int64_t need_total(const unsigned* __restrict__ count) {
  uint64_t v = count[threadIdx.x & 63];
#pragma unroll
  for (int o = 32; o > 0; o >>= 1) v += __shfl_xor(v, o);
  return (int64_t)__builtin_amdgcn_readfirstlane((unsigned)(v & 0xffffffffu)) |
         ((int64_t)__builtin_amdgcn_readfirstlane((unsigned)(v >> 32)) << 32);
}

// x6c_tile_rows with the rows' splits produced per chunk by loadX(q, xa[3]) (for
// operands formed from other data, such as the diagonal model's [x^2, x] features):
// the same products, order and chains, NCH chunks' splits live at a time.
template <int NQ, int MAXCH, typename LX, typename LB>
__device__ __forceinline__ f32x16 x6c_tile_rows_fn(LX loadX, const bf16x8 ones, LB loadB) {
  constexpr int NCH = NQ < MAXCH ? NQ : MAXCH;
  f32x16 acc[NCH];
#pragma unroll
  for (int h = 0; h < NCH; ++h) acc[h] = zero16();
#pragma unroll
  for (int q0 = 0; q0 < NQ; q0 += NCH) {
    bf16x8 b[NCH][4], xa[NCH][3];
#pragma unroll
    for (int h = 0; h < NCH; ++h) {
      if (q0 + h < NQ) {
        loadX(q0 + h, xa[h]);
#pragma unroll
        for (int t = 0; t < 4; ++t) b[h][t] = loadB(q0 + h, t);
      }
    }
    // Chain-major, as x6c_tile.
#pragma unroll
    for (int h = 0; h < NCH; ++h) {
      if (q0 + h < NQ) {
#pragma unroll
        for (int step = 0; step < 7; ++step) {
          const bf16x8 B = step == 0 ? b[h][1] : step == 1 ? b[h][2] : step <= 3 ? b[h][0]
                         : step == 4 ? b[h][1] : step == 5 ? b[h][3] : b[h][0];
          const bf16x8 A = step == 0 ? xa[h][1] : step == 1 ? xa[h][0] : step == 2 ? xa[h][2]
                         : step == 3 ? xa[h][1] : step == 4 ? xa[h][0] : step == 5 ? ones : xa[h][0];
          acc[h] = mfma_bf16(A, B, acc[h]);
        }
      }
    }
  }
  f32x16 t = acc[0];
#pragma unroll
  for (int h = 1; h < NCH; ++h) {
#pragma unroll
    for (int i = 0; i < 16; ++i) t[i] += acc[h][i];
  }
  return t;
}

// ---------------------------------------------------------------------------
// Range-checked buffer loads.  A raw buffer resource covers `bytes` bytes from
// `base`; a lane whose byte offset is at or beyond that reads zero and makes no
// memory access.  Streaming loops use them to issue the same number of load
// instructions in every iteration whatever the data (a row past the slab, a
// log-joint row not needed): the compiler can then count the outstanding loads
// exactly and wait only for the ones an instruction consumes, so prefetches stay
// in flight across iterations.
// ---------------------------------------------------------------------------
typedef __amdgpu_buffer_rsrc_t buf_rsrc;
constexpr int kBufOob = (int)0x80000000u;   // an offset beyond every resource here
constexpr int kBufNt = 2;                   // cache policy: non-temporal (read once)

// A lane's offset, kept in a register as computed: without this the compiler may
// turn `cond ? offset : kBufOob` into a branch around the load, which makes the
// number of loads depend on the path again.
__device__ __forceinline__ int buf_off(int off) {
  asm volatile("" : "+v"(off));
  return off;
}

__device__ __forceinline__ buf_rsrc make_rsrc(const void* base, uint32_t bytes) {
  return __builtin_amdgcn_make_buffer_rsrc(const_cast<void*>(base), (short)0, (int)bytes, 0x00020000);
}

// 16 bytes per lane from a buffer straight into LDS (buffer_load_dwordx4 ... lds):
// lane l's bytes at byte offset voff + soff of the buffer land at dst + 16 l, where
// dst is the wave's LDS base (wave-uniform; it goes to M0).  No registers hold the
// data on the way.  The writes are complete, for the issuing wave, once its
// vector-memory count drains: dma_barrier waits for that before the workgroup
// barrier, and nothing may read the destination before that barrier.
// Issued from inline assembly on purpose: the compiler does not see an LDS store,
// so it does not make every later LDS read wait for the transfer (it cannot tell
// the buffers apart).  Its own vector-memory waits stay correct, since these
// loads only add to the in-order count those waits drain.
typedef __attribute__((address_space(3))) void lds_void_t;
typedef int i32x4_t __attribute__((ext_vector_type(4)));
struct DmaSrc {
  i32x4_t words;
};
__device__ __forceinline__ DmaSrc dma_src(const void* base, uint32_t bytes) {
  const uint64_t a = (uint64_t)base;
  DmaSrc d;
  d.words.x = __builtin_amdgcn_readfirstlane((int)(uint32_t)a);
  d.words.y = __builtin_amdgcn_readfirstlane((int)((uint32_t)(a >> 32) & 0xffffu));
  d.words.z = __builtin_amdgcn_readfirstlane((int)bytes);
  d.words.w = 0x00020000;
  return d;
}
// M0 is the compiler's reserved register, so the asm saves and restores it.
__device__ __forceinline__ void lds_dma16(const DmaSrc& r, void* dst, int voff, int soff) {
  const int lds = __builtin_amdgcn_readfirstlane((int)(uint32_t)(uintptr_t)(lds_void_t*)dst);
  int saved;
  asm volatile("s_mov_b32 %0, m0\n\ts_mov_b32 m0, %1\n\ts_nop 0\n\tbuffer_load_dwordx4 %2, %3, %4 offen lds\n\t"
               "s_mov_b32 m0, %0"
               : "=&s"(saved) : "s"(lds), "v"(voff), "s"(r.words), "s"(soff) : "memory");
}
// Wait until at most N vector-memory operations of the wave are outstanding.
template <int N>
__device__ __forceinline__ void vm_wait() {
  static_assert(N >= 0 && N <= 63, "vmcnt field");
  asm volatile("s_waitcnt vmcnt(%0)" ::"n"(N) : "memory");
}
__device__ __forceinline__ void dma_barrier() {
  asm volatile("s_waitcnt vmcnt(0) lgkmcnt(0)\n\ts_barrier" ::: "memory");
}
template <int AUX = 0>
__device__ __forceinline__ float buf_load_f32(buf_rsrc r, int off) {
  return __builtin_bit_cast(float, __builtin_amdgcn_raw_buffer_load_b32(r, off, 0, AUX));
}
__device__ __forceinline__ unsigned buf_load_u32(buf_rsrc r, int off) {
  return __builtin_amdgcn_raw_buffer_load_b32(r, off, 0, 0);
}
__device__ __forceinline__ double buf_load_f64(buf_rsrc r, int off) {
  return __builtin_bit_cast(double, __builtin_amdgcn_raw_buffer_load_b64(r, off, 0, 0));
}
__device__ __forceinline__ f32x4 buf_load_f32x4(buf_rsrc r, int off) {
  return __builtin_bit_cast(f32x4, __builtin_amdgcn_raw_buffer_load_b128(r, off, 0, 0));
}

// Rows of one slab of X through a resource whose byte 0 is the slab's first row
// (slab_rsrc; the slab spans under 2 GiB, slab_fits).  slab_row4 reads the four floats
// at column d0 of slab row `rel`: zero when !valid and from column D on.  A lane with
// nothing to read gets an offset past the resource, so there is no branch and the loads
// of a sequence stay in flight together; only where D % 4 != 0 (uniform) are the
// columns past D inside the last vector zeroed by selects.
__host__ __device__ inline bool slab_fits(int64_t rows, int64_t ldx) {
  return rows * ldx * (int64_t)sizeof(float) <= ((int64_t)1 << 31) - 256;
}
__device__ __forceinline__ buf_rsrc slab_rsrc(const float* X, int64_t ldx, int64_t r_begin, int64_t r_end) {
  return make_rsrc(X + r_begin * ldx, (uint32_t)((r_end - r_begin) * ldx * (int64_t)sizeof(float)));
}
__device__ __forceinline__ f32x4 slab_row4(buf_rsrc r, int64_t ldx, int rel, int d0, int D, bool valid) {
  const bool in = valid && d0 < D;
  f32x4 v = buf_load_f32x4(r, buf_off(in ? (int)(((int64_t)rel * ldx + d0) * (int64_t)sizeof(float)) : kBufOob));
  if (D & 3) {
    if (d0 + 1 >= D) v.y = 0.0f;
    if (d0 + 2 >= D) v.z = 0.0f;
    if (d0 + 3 >= D) v.w = 0.0f;
  }
  return v;
}

// Workspace cap for the stored log-joint of one call (N/32 x K/32 tiles of 4 KiB).
constexpr size_t kMaxLjBytes = (size_t)16 << 30;

// The log-joint is stored only on request (FGMM_FLAG_STORE_LOGJOINT); RECOMPUTE,
// the default plan, overrides it.
__host__ __device__ constexpr bool wants_stored_lj(unsigned flags) {
  return (flags & FGMM_FLAG_STORE_LOGJOINT) != 0 && (flags & FGMM_FLAG_RECOMPUTE) == 0;
}
// The device-selected stored branch (FGMM_FLAG_STORE_LOGJOINT_AUTO), unless an
// explicit plan flag takes precedence.
__host__ __device__ constexpr bool wants_auto_lj(unsigned flags) {
  return (flags & FGMM_FLAG_STORE_LOGJOINT_AUTO) != 0 &&
         (flags & (FGMM_FLAG_STORE_LOGJOINT | FGMM_FLAG_RECOMPUTE | FGMM_FLAG_BF16)) == 0;
}

// Largest row stride (floats) of X for the buffer-loaded streaming passes: a
// tile's byte offsets (256 rows x stride x 4) must stay below 2^31.
constexpr int64_t kMaxBufLdx = (int64_t)1 << 20;

// Largest N one E-step call takes: pass-1 grids hold N / 128 workgroups, which
// must stay within the 2^31 - 1 grid limit.  Larger data sets stream in chunks.
constexpr int64_t kMaxRows = (int64_t)1 << 37;

// Partial counts from which the reductions use one wave per output element.
constexpr int kWideReduce = 128;

__host__ __device__ constexpr int64_t cdiv(int64_t a, int64_t b) { return (a + b - 1) / b; }
__host__ __device__ constexpr int64_t round_up(int64_t a, int64_t b) { return cdiv(a, b) * b; }

// The stored-log-joint probe (FGMM_FLAG_STORE_LOGJOINT_AUTO): up to kProbeTiles
// 32-row tiles spread over the rows, one count of needed (row, block) pairs per
// tile; at least half of the sampled pairs selects the stored branch.  Up to
// kProbeMaxKB blocks (a probe keeps a tile's block maxima in LDS).
constexpr int kProbeTiles = 64;
constexpr int kProbeMaxKB = 512;
__host__ __device__ constexpr size_t probe_bytes() { return (size_t)kProbeTiles * sizeof(unsigned); }
// What a kernel needs to evaluate the probe's choice (count == nullptr: no probe).
struct ProbeSel {
  const unsigned* count;
  int n;
  int64_t min_pairs;
};
// The stored branch is selected (uniform; false without a probe).
__device__ __forceinline__ bool probe_selects(const ProbeSel& p) {
  if (p.count == nullptr) return false;
  const int lane = threadIdx.x & 63;
  unsigned v = lane < p.n ? p.count[lane] : 0u;
  uint64_t t = v;
#pragma unroll
  for (int o = 32; o > 0; o >>= 1) t += __shfl_xor(t, o);
  const uint64_t tot = (uint64_t)__builtin_amdgcn_readfirstlane((unsigned)t) |
                       ((uint64_t)__builtin_amdgcn_readfirstlane((unsigned)(t >> 32)) << 32);
  return (int64_t)tot >= p.min_pairs;
}
// The sampled tiles (tile s of ntile is s * tiles / ntile) and the probe's
// threshold: half of the sampled (row, block) pairs.
__host__ __device__ inline int64_t probe_tile(int s, int64_t N, int ntile) { return (int64_t)s * cdiv(N, 32) / ntile; }
__host__ inline int64_t probe_min_pairs(int64_t N, int ntile, int KB) {
  int64_t rows = 0;
  for (int s = 0; s < ntile; ++s) {
    const int64_t t = probe_tile(s, N, ntile);
    rows += N - t * 32 < 32 ? N - t * 32 : 32;
  }
  return cdiv(rows * KB, 2);
}

__host__ inline size_t align256(size_t x) { return (x + 255) & ~size_t(255); }

// Compute units of the current device, cached per device (256 on an MI355X; fewer
// in a partitioned mode).  Work splits and workspace sizes derive from it, so a
// workspace query and the call it sizes must run with the same device current.
// Falls back to 256 where no device is visible (host-only size queries).
__host__ inline int current_device_cus() {
  constexpr int kMaxDevices = 64;
  static std::atomic<int> cache[kMaxDevices];
  int dev = 0;
  if (hipGetDevice(&dev) != hipSuccess || dev < 0 || dev >= kMaxDevices) {
    (void)hipGetLastError();
    return 256;
  }
  int v = cache[dev].load(std::memory_order_relaxed);
  if (v <= 0) {
    int cus = 0;
    if (hipDeviceGetAttribute(&cus, hipDeviceAttributeMultiprocessorCount, dev) != hipSuccess || cus <= 0) {
      (void)hipGetLastError();
      cus = 256;
    }
    cache[dev].store(cus, std::memory_order_relaxed);
    v = cus;
  }
  return v;
}

// One step of a gathering pass's row queue (a 64-entry ring in LDS, q_l[pos & 63],
// with qt - qh < 32 rows waiting): w is the need word of tile base / 32 + lane of the
// current batch (0 for words already taken, lanes below jn), nz the ballot of w != 0.
// A first word with 8 or more rows is queued by 32 lanes at once, one row each; a run
// of sparser words is queued in one go, each lane writing the rows of its own word
// after a prefix sum of the counts, as many words as the ring holds.  Either way the
// rows go in tile order and, within a word, in bit order, and qt and jn advance past
// the words taken.
__device__ __forceinline__ void queue_words(unsigned w, uint64_t nz, int base, int lane, int c, int g,
                                            int* q_l, int& qt, int& jn) {
  const int pc = __builtin_popcount(w);
  const uint64_t big = __builtin_amdgcn_ballot_w64(pc >= 8);
  const int j = __builtin_ctzll(nz);
  if ((big >> j) & 1ull) {
    const unsigned m = __builtin_amdgcn_readlane(w, j);
    if (g == 0 && ((m >> c) & 1u)) q_l[(qt + __builtin_popcount(m & ((1u << c) - 1u))) & 63] = base + 32 * j + c;
    qt += __builtin_popcount(m);
    jn = j + 1;
    return;
  }
  // Words before the next dense one; word j (fewer than 8 rows) always fits, since
  // the ring has more than 32 free entries.
  const int lim = big != 0ull ? __builtin_ctzll(big) : 64;
  int incl = pc;
#pragma unroll
  for (int o = 1; o < 64; o <<= 1) {
    const int v = __shfl_up(incl, o);
    if (lane >= o) incl += v;
  }
  const bool take = lane >= jn && lane < lim && incl <= 64 - 32;
  const uint64_t tm = __builtin_amdgcn_ballot_w64(take);
  const int jl = 64 - __builtin_clzll(tm);
  if (take) {
    unsigned m = w;
    int pos = qt + incl - pc;
    while (m != 0u) {
      q_l[pos & 63] = base + 32 * lane + __builtin_ctz(m);
      ++pos;
      m &= m - 1u;
    }
  }
  qt += __builtin_amdgcn_readlane(incl, jl - 1);
  jn = jl;
}

// Fill a gathering pass's row queue until 32 rows wait or the slab's tiles run out.
// words(tb) loads the need word of tile tb + lane (0 past the slab); mword holds the
// current batch of 64 words, mnext the next, jn the first word not yet taken.  PAR
// selects queue_words' prefix-sum step; without it one word is queued per step (for
// kernels whose registers are too tight for the prefix sum).
template <bool PAR, typename Words>
__device__ __forceinline__ void queue_fill(Words words, int64_t& tb, int64_t t_begin, int64_t t_end,
                                           unsigned& mword, unsigned& mnext, int& jn, int& qt, int qh,
                                           int lane, int c, int g, int* q_l) {
  while (qt - qh < 32) {
    const unsigned w = (PAR && lane >= jn) ? mword : 0u;
    const uint64_t live = jn >= 64 ? 0ull : (~0ull << jn);
    const uint64_t nz = PAR ? __builtin_amdgcn_ballot_w64(w != 0u) : __builtin_amdgcn_ballot_w64(mword != 0u) & live;
    if (nz == 0) {
      tb += 64;
      if (tb >= t_end) break;
      mword = mnext;
      mnext = words(tb + 64);
      jn = 0;
      continue;
    }
    if constexpr (PAR) {
      queue_words(w, nz, (int)(tb - t_begin) * 32, lane, c, g, q_l, qt, jn);
    } else {
      const int j = __builtin_ctzll(nz);
      const unsigned m = __builtin_amdgcn_readlane(mword, j);
      const int base = (int)((tb + j - t_begin) * 32);
      if (g == 0 && ((m >> c) & 1u)) q_l[(qt + __builtin_popcount(m & ((1u << c) - 1u))) & 63] = base + c;
      qt += __builtin_popcount(m);
      jn = j + 1;
    }
  }
}

// Gathering passes: one workgroup of W waves per (slab group of W row slabs,
// component or component block), workgroup b running on XCD b % 8.  With 8 or more
// slab groups each XCD serves whole groups, so all components of a group share that
// XCD's L2 for the rows of X; with fewer, the XCDs that share a group split its
// components (x % G serves group x % G, taking every c-th component).  The slab count
// is rounded so that the group count is 1, 2, 4 or a multiple of 8: every XCD then
// gets the same work.
__host__ inline int64_t gather_slab_count(int64_t want, int64_t max_slabs, int W) {
  const int64_t groups = cdiv(want < 1 ? 1 : want, W);
  const int64_t g = groups <= 1 ? 1 : groups <= 2 ? 2 : groups <= 4 ? 4 : round_up(groups, 8);
  const int64_t n = g * W;
  return n < max_slabs ? n : max_slabs;
}
// The gathering passes read a slab's row state (logZ2, and ||x||^2 for the isotropic
// model) through one buffer resource whose byte offsets are 32-bit: a slab holds at
// most this many rows, so the offsets stay below 2^31 whatever N and K are (beyond
// it the plan takes more slabs).  Rounded down to whole 32-row tiles.
__host__ inline int64_t max_slab_rows(size_t state_bytes_per_row) {
  return ((((int64_t)1 << 31) - 256) / (int64_t)state_bytes_per_row) / 32 * 32;
}
__host__ inline int64_t cap_slab_rows(int64_t rows_per_slab, size_t state_bytes_per_row) {
  const int64_t cap = max_slab_rows(state_bytes_per_row);
  return rows_per_slab < cap ? rows_per_slab : cap;
}
__host__ inline int64_t gather_item_grid(int G, int K) {
  if (G >= 8) return cdiv(G, 8) * (int64_t)K * 8;
  return 8 * cdiv(K, 8 / (G < 1 ? 1 : G));
}
// (slab group sg, component k) of workgroup b; false for a workgroup with no item.
__device__ __forceinline__ bool gather_item(unsigned b, int G, int K, int& sg, int& k) {
  const int x = (int)(b & 7u), i = (int)(b >> 3);
  if (G >= 8) {
    k = i % K;
    sg = (i / K) * 8 + x;
    return sg < G;
  }
  sg = x % G;
  const int c = (8 - sg + G - 1) / G;   // XCDs serving group sg
  k = x / G + i * c;
  return k < K;
}

}  // namespace fgmm
