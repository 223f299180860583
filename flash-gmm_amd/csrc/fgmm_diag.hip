// Diagonal-covariance GMM E-step for gfx950.
//
// Math (reference: flash_gmm_diag_h100.py:332-340 constants, :116-119 log-joint,
// :250-260 accumulation, :380-384 outputs), in log2 units with
//   w_kd = 0.5 * exp(-lss_kd) * log2(e),   v_kd = mu_kd * w_kd,
//   C_k  = (lpi_k - 0.5*(D*log(2pi) + sum_d lss_kd)) * log2(e) - sum_d mu_kd^2 w_kd:
//   ll2_nk = C_k + [x_n^2, x_n] . [-w_k, 2 v_k]          (one contraction over 2D features)
//   r_nk = 2^(ll2_nk - logZ2_n)
//   Nk_k = sum_n r_nk;  mu_acc_kd = sum_n r_nk x_nd;  rxsq_kd = sum_n r_nk x_nd^2
//   sig_acc_kd = rxsq_kd - 2 mu_kd mu_acc_kd + mu_kd^2 Nk_k   (fp64, in the finish)
//
// Same structure as the isotropic kernels (fgmm_iso.hip):
//   diag_x6_prep      O(K*D): the feature operand [-w, 2v] as three-way bf16 splits with
//                     per-chunk centring offsets in matrix-core operand order, and C'_k.
//   diag_lse_x6       pass 1 up to D = 128 with the rows' split features resident in
//                     registers (the x^2 half formed on the fly), the centred
//                     split-bf16 contraction, online log-sum-exp, need masks per half
//                     block (16 components) or the stored log-joint.
//   diag_lse_ctile    pass 1 above D = 128 (any D), tiled over components as well.
//   diag_accum_gather pass 2 of the default plan up to D = 128: the needed rows of each
//                     slab, the log-joint recomputed bit for bit as pass 1 forms it,
//                     r^T [X | X^2] as six split-bf16 products per 16 rows.
//   diag_accum_drange pass 2 of the default plan above D = 128, per dimension range.
//   diag_accum_sparse / diag_accum_lj2 / diag_accum_lj
//                     pass 2 of the stored plan (FGMM_FLAG_STORE_LOGJOINT, D <= 256).
//   diag_reduce       fixed-order fp64 sum of the slab partials and the sig identity.
//   diag_bf16_*       the bf16 operand contract (FGMM_FLAG_BF16).
// Row slabs are disjoint ([s*R, min(N, (s+1)*R))), so no row is counted twice at a
// slab boundary.

#include "fgmm_common.hpp"

#include <math.h>

#include <algorithm>
#include <type_traits>

namespace fgmm {
namespace {

constexpr int kWaves = 4;
constexpr int kThreads = 64 * kWaves;
constexpr int kAccWaves = 8;
constexpr int kAccThreads = 64 * kAccWaves;

constexpr size_t kMaxLds = 160 * 1024;

// D padded to a multiple of 32 up to 128, of 64 above (where pass 1 tiles the
// contraction over components and pass 2 splits r^T [X | X^2] over dimension ranges:
// each of the four accumulation chains then gets the same number of chunks).
__host__ inline int diag_padded_dim(int64_t D) {
  return D <= 128 ? (int)round_up(D < 1 ? 1 : D, 32) : (int)round_up(D, 64);
}
constexpr int kCtWaves = 4;                               // waves per workgroup, one per SIMD
constexpr int kGatherWaves = 4;                           // waves (row slabs) per gathering workgroup
constexpr int kCtChains = 4;                              // accumulation chains (chunk q -> q % 4)
constexpr int kDrange = 1024;                             // dimensions of r^T [X | X^2] per pass-2 workgroup
constexpr int kDrTiles = kDrange / 32 / kCtWaves;         // 32-column tiles per pass-2 wave
// Component blocks per pass-1 tile: two (two waves per SIMD) up to D = 1024, four
// (one wave per SIMD) above.
__host__ __device__ constexpr int ctile_blocks(int DP) { return DP <= 1024 ? 2 : 4; }
__host__ __device__ constexpr int ctile_stage_ops(int CTB) { return CTB * 2 * 4 * 64; }   // bf16x8 per two-chunk stage
__host__ __device__ constexpr size_t lse_ctile_base(int CTB) {
  return (size_t)2 * ctile_stage_ops(CTB) * sizeof(bf16x8) + (size_t)2 * CTB * 32 * sizeof(double);
}
// Component blocks whose half-block need bounds (bf16, 2 x 32 rows per wave) fit
// beside the stages.
__host__ __device__ constexpr int ctile_need_exact_cap(int CTB) {
  return (int)((kMaxLds - lse_ctile_base(CTB)) / (kCtWaves * 2 * 32 * 2));
}
// fp32 row stride of the X tile: rows 8 apart (the lane-halves of a B operand) and the
// 16-byte row writes fall in distinct banks.
__host__ __device__ constexpr int drange_rs(int DR) { return DR + 4; }
__host__ __device__ constexpr size_t accum_drange_lds_bytes(int DR) {
  return (size_t)32 * drange_rs(DR) * sizeof(float)         // X of 32 rows
         + (size_t)kCtWaves * 16 * 64 * sizeof(float)        // the four chains of S
         + (size_t)32 * sizeof(double)                       // logZ2 of the rows
         + (size_t)kCtWaves * 64 * sizeof(int);              // row queue per wave
}

__host__ __device__ constexpr size_t bf16_lse_lds_base(int DP) {
  return (size_t)2 * (DP / 8) * 64 * 16 + (size_t)2 * 32 * sizeof(float);   // feature blocks and c0
}
// bf16 operand contract (defined with its kernels below).  Above D = 256 it stores
// the log-joint ([32-row tile][KP][32 rows], fp32).
constexpr int kBwCB = 8;     // component blocks per wide bf16 pass-2 workgroup (one per wave)
constexpr int kBwDR = 128;   // dimensions per wide bf16 pass-2 workgroup
__host__ __device__ constexpr bool diag_bf16_wide(int DP) { return DP > 256; }
__host__ inline size_t bw_lj_bytes(int64_t N, int KP) {
  return (size_t)round_up(cdiv(N, 32), 4) * (size_t)KP * 32 * sizeof(float);
}
__host__ __device__ constexpr int bf16_parts(int DP);
__host__ __device__ constexpr size_t bf16_accum_lds_bytes(int DP, int CB);
__host__ inline int bf16_blocks_per_group(int DP, int KB);
__host__ __device__ constexpr int bf16_row_partials(int DP, int CB);

// Pass 1 keeps the rows' split features in registers (diag_lse_x6) up to D = 128.
__host__ __device__ constexpr bool diag_uses_x6(int DP) { return DP <= 128; }

// The stored branch of FGMM_FLAG_STORE_LOGJOINT_AUTO (default plan, D <= 96): pass 1
// keeps every log-joint tile (row-major, as the stored plan's), the rows' features
// [x^2 | x] in three bf16 parts (row stride ljd_rs, chunk q at columns 16q .. 16q + 15
// in pass 1's order) and logZ2 as (hi, lo) float pairs; diag_accum_ljt streams them.
__host__ __device__ constexpr int ljd_rs(int DP) { return 2 * DP + 16; }
__host__ __device__ constexpr size_t ljd_xsplit_bytes(int DP) { return (size_t)3 * 32 * ljd_rs(DP) * 2; }
__host__ __device__ constexpr bool ljd_applies(int DP) { return DP <= 96; }
// Piece (16 bytes) swizzle of a 32 x 16 float transposition tile: row r's piece p sits
// at p ^ ljd_swz(r), so that the column writes and the row reads of a wave fall in
// distinct banks.
__device__ __forceinline__ int ljd_swz(int r) { return (((r >> 2) & 1) << 1) | (((r >> 1) ^ (r >> 3)) & 1); }

struct DiagPlan {
  int64_t N, K, D;
  int DP, FP;   // D padded (32 up to 128, then 64); feature count 2*DP
  int KB, KP;
  int cpg;      // component blocks per pass-2 workgroup
  int ncg, nslab, rgroups, npart;
  int64_t rows_per_slab;
  bool bf16;    // bf16 operand contract (FGMM_FLAG_BF16)
  bool lj;      // pass 1 stores the log-joint; pass 2 reads it
  int lj_nh;    // column parts per component block in that pass 2 (1 or 2)
  bool lj_sparse;   // the stored log-joint in the sparse form (D <= 128)
  bool need;        // default plan: pass 1 leaves need masks, pass 2 gathers the needed rows
  bool ctile;       // above D = 128: component-tiled pass 1 (both plans), range pass 2 (default)
  bool rexact;      // need masks from block maxima kept in LDS (else the running-max bound)
  int ndr;          // dimension ranges of the range pass 2 (and of the wide bf16 pass 2)
  bool bfw;         // bf16 contract above D = 256: stored log-joint, diag_bf16_*_wide
  bool bfneed;      // bf16 contract up to D = 128: need masks from pass 1, diag_bf16_gather in pass 2
                    // (or diag_bf16_accum where most pairs are needed)
  bool autolj;      // the default plan with a stored branch that a row-sample probe selects on the
                    // device (FGMM_FLAG_STORE_LOGJOINT_AUTO, D <= 96)
  int nprobe;       // the probe's sampled tiles
  size_t off_xsplit, off_zpair, off_probe;
  size_t off_musw, off_mu3, off_kcx6, off_kcx6lin, off_kclin, off_rowstat, off_part_mu,
      off_part_sq, off_part_nk, off_lj, off_ljmax, off_ljmask, off_ljcount, total;
};

// Bytes of LDS the split-bf16 pass 1 uses at width DP (x6_lds_bytes, for the host).
__host__ size_t x6_lds_bytes_rt(int DP);

// Pass 1 with need masks keeps a bf16 bound of each row's half-block maximum in LDS,
// 2 bytes per (row, block) for each of its 8 waves, up to the LDS left in a compute
// unit; beyond that many blocks the masks come from the running-max bound.
__host__ inline int need_exact_cap(int DP) {
  const size_t base = x6_lds_bytes_rt(DP);
  return base >= 160 * 1024 ? 0 : (int)((160 * 1024 - base) / (8 * 32 * 2));
}

// Pass 2 reads the stored log-joint when it is requested, there are at least 4
// component blocks, 32 < D <= 256 (above, only the default plan has kernels), and
// the tiles (one per pass-1 wave) fit under kMaxLjBytes.  At D <= 32 nearly every row of a tile is needed and
// recomputing the short contraction costs less than the traffic (N=1M, K=1024:
// 3.67 ms recomputed, 4.12 ms stored).
__host__ inline bool use_stored_lj(int64_t N, int KB, int DP, bool allow) {
  return allow && KB >= 4 && DP > 32 && DP <= 256 &&
         (size_t)round_up(cdiv(N, 32), 4) * (size_t)KB * kLjTile * sizeof(float) <= kMaxLjBytes;
}

DiagPlan make_plan(int64_t N, int64_t K, int64_t D, bool allow_lj = false, bool bf16 = false,
                   bool auto_lj = false) {
  DiagPlan p{};
  p.N = N; p.K = K; p.D = D;
  p.DP = diag_padded_dim(D);
  p.FP = 2 * p.DP;
  p.KB = (int)cdiv(K, 32);
  p.KP = p.KB * 32;
  p.bf16 = bf16;
  p.lj = !bf16 && use_stored_lj(N, p.KB, p.DP, allow_lj);
  p.need = !bf16 && !p.lj;
  p.autolj = p.need && auto_lj && ljd_applies(p.DP) && N > 0 && p.KB > 0 && p.KB <= kProbeMaxKB &&
             (size_t)round_up(cdiv(N, 32), 4) * (size_t)p.KB * kLjTile * sizeof(float) <= kMaxLjBytes;
  p.nprobe = p.autolj ? (int)std::min<int64_t>(kProbeTiles, cdiv(N, 32)) : 0;
  p.ctile = !bf16 && !diag_uses_x6(p.DP);
  p.rexact = p.need && p.KB <= (p.ctile ? ctile_need_exact_cap(ctile_blocks(p.DP)) : need_exact_cap(p.DP));
  p.ndr = p.ctile ? (int)cdiv(p.DP, kDrange) : 1;
  p.bfw = bf16 && diag_bf16_wide(p.DP);
  if (p.bfw) {
    p.cpg = kBwCB;
    p.rgroups = 1;
    p.ndr = (int)cdiv(p.DP, kBwDR);
  } else if (bf16) {
    p.cpg = bf16_blocks_per_group(p.DP, p.KB);
    p.rgroups = bf16_row_partials(p.DP, p.cpg);
  } else if (p.lj) {
    // 8 component blocks per workgroup, or 4 for K <= 224.  Two waves share a
    // block (one half of the columns each) where one wave's x and x^2
    // accumulators would not fit: above D = 128, or at D = 128 with 4 blocks.
    p.cpg = (p.KB >= 8 && p.DP <= 128) ? 8 : 4;
    p.lj_nh = (p.DP > 128 || (p.DP == 128 && p.cpg == 4)) ? 2 : 1;
    p.rgroups = kAccWaves / (p.cpg * p.lj_nh);
  } else {
    p.cpg = 1;        // one wave (D <= 128) or workgroup per (row slab, component block)
    p.rgroups = 1;
  }
  p.ncg = (int)cdiv(p.KB, p.cpg);
  const int64_t tile_rows = 32 * (bf16 && !p.bfw ? kAccWaves / (p.cpg * bf16_parts(p.DP)) : p.rgroups);
  if (p.bfw && N > 0 && p.KB > 0) {
    // About two workgroups per compute unit.
    int64_t want = cdiv((int64_t)2 * current_device_cus(), (int64_t)p.ncg * p.ndr);
    if (want > cdiv(N, 32)) want = cdiv(N, 32);
    p.rows_per_slab = round_up(cdiv(N, want), 32);
    p.nslab = (int)cdiv(N, p.rows_per_slab);
  } else if (p.need && p.ctile && N > 0 && p.KB > 0) {
    // One 4-wave workgroup per (slab, block, dimension range) and compute unit (its
    // X tile takes most of the LDS): about two rounds of workgroups.
    int64_t want = cdiv((int64_t)2 * current_device_cus(), (int64_t)p.KB * p.ndr);
    const int64_t max_slabs = cdiv(N, 32);
    if (want > max_slabs) want = max_slabs;
    p.rows_per_slab = cap_slab_rows(round_up(cdiv(N, want), 32), sizeof(double));
    p.nslab = (int)cdiv(N, p.rows_per_slab);
  } else if (p.need && N > 0 && p.KB > 0) {
    // The gathering pass 2: eight waves per compute unit, two rounds at one wave per
    // SIMD (one round where two fit).
    const int64_t want = gather_slab_count(cdiv((int64_t)8 * current_device_cus(), p.KB), cdiv(N, 32), kGatherWaves);
    p.rows_per_slab = cap_slab_rows(round_up(cdiv(N, want), 32), sizeof(double));
    p.nslab = (int)cdiv(N, p.rows_per_slab);
  } else if (N > 0 && p.ncg > 0) {
    int64_t want = (int64_t)current_device_cus() / p.ncg;
    if (want >= 8) want = (want / 8) * 8;
    if (want < 1) want = 1;
    const int64_t max_slabs = cdiv(N, tile_rows);
    if (want > max_slabs) want = max_slabs;
    p.rows_per_slab = round_up(cdiv(N, want), tile_rows);
    p.nslab = (int)cdiv(N, p.rows_per_slab);
  } else {
    p.rows_per_slab = tile_rows;
    p.nslab = 0;
  }
  p.npart = p.nslab * p.rgroups;
  size_t off = 0;
  // The bf16 contract's operands and constants; the fp32 plans' split operands.
  p.off_musw = off;    off = align256(off + (bf16 ? (size_t)p.KP * p.FP * sizeof(float) : 0));
  p.off_kclin = off;   off = align256(off + (bf16 ? (size_t)p.KP * sizeof(double) : 0));
  p.off_mu3 = off;     off = align256(off + (bf16 ? 0 : (size_t)p.KP * (p.DP / 8) * 4 * 2 * sizeof(bf16x8)));
  p.off_kcx6 = off;    off = align256(off + (bf16 ? 0 : (size_t)p.KP * sizeof(double)));
  p.off_kcx6lin = off; off = align256(off + (bf16 ? 0 : (size_t)p.KP * sizeof(double)));
  p.off_rowstat = off; off = align256(off + (size_t)(N > 0 ? N : 0) * sizeof(double));
  p.off_part_mu = off; off = align256(off + (size_t)p.npart * p.KP * p.DP * sizeof(float));
  p.off_part_sq = off; off = align256(off + (size_t)p.npart * p.KP * p.DP * sizeof(float));
  p.off_part_nk = off; off = align256(off + (size_t)p.npart * p.KP * sizeof(float));
  // One log-joint tile per pass-1 wave (the grid's 32-row tiles, rounded up to 4);
  // in the sparse form with each row's block maxima and the need masks, one half
  // (16 components) per pass-1 wave.
  // The default plan keeps the need masks only: two words (one per half block) per
  // (32-row tile, block), ORed by pass 2.
  p.lj_sparse = p.lj && diag_uses_x6(p.DP);
  const size_t ntile = (p.lj || p.need) ? (size_t)round_up(cdiv(N, 32), 4) * p.KB : 0;
  // The bf16 contract's need masks (one word per (tile, block)): each row's block maxima
  // (bf16, 2 bytes per row and block for the 4 waves of a pass-1 workgroup) in LDS.
  p.bfneed = bf16 && !p.bfw && p.DP <= 128 && p.KB > 0 &&
             bf16_lse_lds_base(p.DP) + (size_t)kWaves * 32 * p.KB * 2 <= kMaxLds;
  const size_t nsp = (p.lj_sparse || p.need || p.bfneed) ? (p.bfneed ? (size_t)round_up(cdiv(N, 32), 4) * p.KB : ntile) : 0;
  p.off_lj = off;
  off = align256(off + (p.bfw ? bw_lj_bytes(N, p.KP) : (p.lj || p.autolj) ? ntile * kLjTile * sizeof(float) : 0));
  p.off_ljmax = off;   off = align256(off + (p.lj_sparse ? nsp * 64 * sizeof(float) : 0));
  p.off_ljmask = off;  off = align256(off + nsp * sizeof(uint2));
  p.off_ljcount = off; off = align256(off + ((p.lj_sparse || p.bfneed) ? 64 * sizeof(unsigned) : 0));
  // The stored branch's feature parts and logZ2 pairs (one per pass-1 tile) and the
  // probe's counts.
  const size_t ptiles = p.autolj ? (size_t)round_up(cdiv(N, 32), 4) : 0;
  p.off_xsplit = off;  off = align256(off + ptiles * ljd_xsplit_bytes(p.DP));
  p.off_zpair = off;   off = align256(off + ptiles * 32 * sizeof(float2));
  p.off_probe = off;   off = align256(off + (p.autolj ? probe_bytes() : 0));
  p.total = off;
  return p;
}

__device__ __forceinline__ f32x4 sq4(f32x4 v) { return v * v; }

// ---------------------------------------------------------------------------
// Pass 1 on the bf16 matrix cores, up to D = 128: the centred split-bf16 cross term
// of the isotropic pass 1 (x6c_tile) over chunks of 8 dimensions.  Chunk q is 16
// features: lane-half g holds dimensions 8q + 4g .. +3 as [x^2 (4), x (4)] against
// [-w (4), 2v (4)], each fp32 value split exactly into three bf16.  The chunk's
// centring offset is o_q = fp32(sum over its 8 dimensions of mu_d^2 w_d), so for
// the components near a row the chunk sum -sum (x_d - mu_d)^2 w_d stays small; the
// offsets return through C'_k = C_k + sum_q o_q in fp64.  CPU emulation of the
// matrix-step rounding on the N=1M, K=1024, D=96 clustered data: max logZ error
// 2.4e-5 over 16,384 rows, against 5.2e-5 for the fp32-step form.
//
// Eight waves = 4 row groups x 2 halves of the chunks, so each wave holds the bf16
// splits of half of its 32 rows' features (72 registers at D = 96).  The two waves
// of a row group then share the rest evenly: each sends the other the fp32 chunk
// sums of the 8 accumulator registers the other owns (through LDS), adds the pair
// for its own 8 (fp32 addition commutes, so the sum does not depend on which wave
// forms it) and runs the online log-sum-exp and the log-joint stores for them; the
// two partial (max, sum) pairs of a row are merged once at the end.
// ---------------------------------------------------------------------------
template <int DP>
constexpr size_t x6_block_bytes() { return (size_t)(DP / 8) * 4 * 64 * sizeof(bf16x8); }
template <int DP>
constexpr int x6_mu_buffers() {
  constexpr size_t ex = (size_t)kWaves * 16 * 64 * sizeof(float);
  return 2 * x6_block_bytes<DP>() + 2 * ex + 3 * 32 * sizeof(double) <= kMaxLds ? 2 : 1;
}
template <int DP>
constexpr size_t x6_lds_bytes() {
  constexpr int MB = x6_mu_buffers<DP>();
  return (size_t)MB * x6_block_bytes<DP>() + (size_t)MB * kWaves * 16 * 64 * sizeof(float) +
         (size_t)(MB + 1) * 32 * sizeof(double);
}

// Prologue of that pass: the split operands [kb][chunk][split 0..2, offset][lane] and
// C'_k in the accumulator's row order.  One 64-thread block per 32 components.
__global__ __launch_bounds__(64) void diag_x6_prep(const float* __restrict__ mu, int64_t ldmu,
                                                   const float* __restrict__ lss, int64_t ldlss, int64_t K,
                                                   int D, int DP, const float* __restrict__ lpi,
                                                   bf16x8* __restrict__ mu3, double* __restrict__ kc_x6,
                                                   double* __restrict__ kc_x6lin, unsigned* __restrict__ ljcount) {
  __shared__ double sC[32];
  const int kb = blockIdx.x;
  const int lane = threadIdx.x, c = lane & 31, g = lane >> 5;
  // Pass 1 counts the needed row pairs of the sparse log-joint into these.
  if (ljcount && kb == 0) ljcount[lane] = 0u;
  const int64_t comp = (int64_t)kb * 32 + c;
  const bool valid = comp < K;
  const int NQ = DP / 8;
  double osum = 0.0;
  for (int q = 0; q < NQ; ++q) {
    f32x4 fw = zero4(), fv = zero4();
    double o = 0.0;
    if (valid) {
#pragma unroll 8
      for (int d = 8 * q; d < 8 * q + 8 && d < D; ++d) {
        const double m = (double)mu[comp * ldmu + d];
        const double w = 0.5 * exp(-(double)lss[comp * ldlss + d]) * kLog2e;
        o = fma(m * m, w, o);
        const int e = d - 8 * q - 4 * g;
        if (e >= 0 && e < 4) {
          fw[e] = (float)(-w);
          fv[e] = (float)(2.0 * m * w);
        }
      }
    }
    bf16x8 s[3];
    split3_bf16(fw, fv, s);
    bf16x8* dst = mu3 + ((int64_t)kb * NQ + q) * 4 * 64 + lane;
#pragma unroll
    for (int t = 0; t < 3; ++t) dst[t * 64] = s[t];
    const float of = (float)o;
    osum += (double)of;
    f32x4 ov = zero4();
    if (g == 0) ov.x = -of;
    bf16x8 so[3];
    split3_bf16(ov, zero4(), so);
    bf16x8 off;
#pragma unroll
    for (int e = 0; e < 8; ++e) off[e] = (__bf16)0.0f;
    if (g == 0) {
      off[0] = so[0][0];
      off[1] = so[1][0];
      off[2] = so[2][0];
    }
    dst[3 * 64] = off;
  }
  if (g == 0) {
    double C = -INFINITY;
    if (valid) {
      double lsum = 0.0, qs = 0.0;
#pragma unroll 8
      for (int d = 0; d < D; ++d) {
        const double l = (double)lss[comp * ldlss + d];
        const double m = (double)mu[comp * ldmu + d];
        lsum += l;
        qs = fma(m * m, 0.5 * exp(-l) * kLog2e, qs);
      }
      C = ((double)lpi[comp] - 0.5 * ((double)D * kLog2Pi + lsum)) * kLog2e - qs + osum;
    }
    sC[c] = C;
    kc_x6lin[comp] = C;   // component order, for the gathering pass 2
  }
  __syncthreads();
  if (lane < 32) {
    const int i = lane & 15, gg = lane >> 4;
    kc_x6[(int64_t)kb * 32 + gg * 16 + i] = sC[acc_row(i, gg)];
  }
}

// What pass 1 leaves for pass 2 besides logZ2.
constexpr int kLjmStore = 1;   // the stored log-joint, its half-block maxima and need masks
constexpr int kLjmNeed = 2;    // need masks only (the default plan)

template <int DP, int LJM, bool ST = false>
__global__ __attribute__((amdgpu_flat_work_group_size(kAccThreads, kAccThreads), amdgpu_waves_per_eu(2, 2)))
void diag_lse_x6(const float* __restrict__ X, int64_t ldx, int64_t N, int D,
                 const bf16x8* __restrict__ mu3, const double* __restrict__ kc_x6, int KB,
                 float* __restrict__ logZ, double* __restrict__ rowstat, float* __restrict__ lj,
                 float* __restrict__ ljmax, unsigned* __restrict__ ljmask, unsigned* __restrict__ ljcount,
                 int dense, int rexact, ProbeSel probe, float* __restrict__ ljd, __bf16* __restrict__ xsplit,
                 float2* __restrict__ zpair) {
  constexpr bool LJ = LJM == kLjmStore;
  constexpr int NQ = DP / 8;              // chunks of 8 dimensions (16 features)
  constexpr int NQH = NQ / 2;             // per half
  constexpr int BLK = NQ * 4 * 64;        // bf16x8 per 32-component block
  constexpr int LPT = BLK / kAccThreads;
  constexpr int MB = x6_mu_buffers<DP>();
  constexpr int NKC = MB + 1;             // constant buffers
  static_assert(BLK % kAccThreads == 0 && NQ % 2 == 0, "split shape");

  extern __shared__ __align__(16) unsigned char lds_raw[];
  unsigned char* p = lds_raw;
  bf16x8* mu_l = reinterpret_cast<bf16x8*>(p); p += (size_t)MB * BLK * sizeof(bf16x8);
  float* ex = reinterpret_cast<float*>(p);     p += (size_t)MB * kWaves * 16 * 64 * sizeof(float);
  double* kc_l = reinterpret_cast<double*>(p);
  // Need masks: each wave's half-block maximum bounds, [wave][block][row] (rexact).
  unsigned short* rmax_l = reinterpret_cast<unsigned short*>(lds_raw + x6_lds_bytes<DP>());

  const int tid = threadIdx.x, lane = tid & 63;
  const int wave = __builtin_amdgcn_readfirstlane(tid >> 6);
  const int c = lane & 31, g = lane >> 5;
  const int rg = wave & 3, h = wave >> 2;
  const int64_t tile = (int64_t)blockIdx.x * kWaves + rg;   // 32-row tile
  const int64_t row = tile * 32 + c;
  const bool valid = row < N;
  // The stored branch of FGMM_FLAG_STORE_LOGJOINT_AUTO (default plan) is the ST
  // instance: it also writes every log-joint tile, the rows' feature parts and logZ2
  // pairs for diag_accum_ljt.  Both instances are launched; the probe's counts let
  // one of them run.
  static_assert(!ST || LJM == kLjmNeed, "the stored branch is the default plan's");
  if (probe.count != nullptr && probe_selects(probe) != ST) return;

  // Blocks go global -> registers -> LDS.  Up to D = 96 through two register
  // stages: block kb + 2 is fetched while block kb is contracted and lands in LDS at
  // the end of iteration kb + 1, so each fetch has a whole iteration to arrive.  At
  // D = 128 (registers) one stage: block kb + 1 is fetched and committed in
  // iteration kb.
  constexpr int NST = DP <= 96 ? 2 : 1;
  bf16x8 st[NST][LPT];
  double kst[NST];
#pragma unroll
  for (int u = 0; u < NST; ++u) kst[u] = 0.0;
  auto fetch = [&](int kb, bf16x8 (&s)[LPT], double& k) {
    if (kb >= KB) return;
    const bf16x8* src = mu3 + (int64_t)kb * BLK;
#pragma unroll
    for (int q = 0; q < LPT; ++q) s[q] = src[q * kAccThreads + tid];
    if (tid < 32) k = kc_x6[(int64_t)kb * 32 + tid];
  };
  auto commit = [&](int kb, const bf16x8 (&s)[LPT], double k) {
    bf16x8* dst = mu_l + (MB == 2 ? (kb & 1) : 0) * BLK;
#pragma unroll
    for (int q = 0; q < LPT; ++q) dst[q * kAccThreads + tid] = s[q];
    if (tid < 32) kc_l[(kb % NKC) * 32 + tid] = k;
  };
  fetch(0, st[0], kst[0]);
  // This half's chunks: dimensions 8q + 4g .. +3 as [x^2, x], split three ways.
  bf16x8 xb[NQH][3];
#pragma unroll
  for (int qq = 0; qq < NQH; ++qq) {
    const f32x4 x = load_row4(X, ldx, row, 8 * (h * NQH + qq) + 4 * g, D, valid);
    split3_bf16(x * x, x, xb[qq]);
  }
  const bf16x8 ones = x6c_ones(lane);
  commit(0, st[0], kst[0]);
  if constexpr (NST == 2) fetch(1, st[NST - 1], kst[NST - 1]);
  lds_barrier();

  double mx = -INFINITY;
  float sm = 0.0f;
  float run_max = -INFINITY;   // running max of the stored log-joint this wave covers
  // The loop is compiled once per half so that register indices stay constant, and
  // unrolled by two so that the staging registers have fixed parity.
  auto run = [&](auto half) {
    constexpr int H = decltype(half)::value;
    constexpr int ib = 8 * H;   // this wave's accumulator registers ib .. ib + 7
    auto step = [&](int kb, auto par) {
      constexpr int P = decltype(par)::value;   // kb & 1
      const int buf = MB == 2 ? P : 0;
      const bool more = kb + 1 < KB;
      constexpr int SN = NST == 2 ? 1 - P : 0;   // stage holding block kb + 1
      if constexpr (NST == 2) {
        fetch(kb + 2, st[P], kst[P]);
      } else {
        fetch(kb + 1, st[0], kst[0]);
      }
      const bf16x8* mp = mu_l + buf * BLK + H * NQH * 4 * 64 + lane;
      // Two accumulator chains (CPU emulation: as accurate as four here, 32 fewer adds).
      const f32x16 xm = x6c_tile<NQH, 2>([&](int q, int t) { return mp[(q * 4 + t) * 64]; }, xb, ones);
      // Slot (buf, rg, H) carries this wave's sums for the other wave's registers.
      float* exw = ex + ((size_t)(buf * kWaves + rg) * 2 + H) * 8 * 64 + lane;
      const float* exr = ex + ((size_t)(buf * kWaves + rg) * 2 + (1 - H)) * 8 * 64 + lane;
#pragma unroll
      for (int j = 0; j < 8; ++j) exw[j * 64] = xm[8 * (1 - H) + j];
      if (MB == 2 && more) commit(kb + 1, st[SN], kst[SN]);
      lds_barrier();
      if (MB == 1 && more) commit(kb + 1, st[SN], kst[SN]);
      const double* kp = kc_l + (kb % NKC) * 32 + g * 16 + ib;
      double ll[8];
      double bm = -INFINITY;
#pragma unroll
      for (int j = 0; j < 8; ++j) {
        ll[j] = kp[j] + (double)(xm[ib + j] + exr[j * 64]);
        bm = fmax(bm, ll[j]);
      }
      const double mn = fmax(mx, bm);
      const double ms = (mn == -INFINITY) ? 0.0 : mn;
      float acc = sm * fast_exp2((float)(mx - ms));
#pragma unroll
      for (int j = 0; j < 8; ++j) acc += fast_exp2((float)(ll[j] - ms));
      sm = acc;
      mx = mn;
      if constexpr (ST) {
        // This wave's 16 components of the 32 rows, row-major into the tile's columns
        // 16H .. 16H + 15, transposed through the exchange slot just read (exr's: its
        // writer, the other wave, writes it again only after the next barrier).  A
        // lane holds local columns 4g .. 4g + 3 (ll[0..3]) and 8 + 4g .. (ll[4..7]);
        // the 16-byte pieces of row r sit at piece p ^ ljd_swz(r).
        float* tl = ex + ((size_t)(buf * kWaves + rg) * 2 + (1 - H)) * 8 * 64;
        const int sw = ljd_swz(c);
        *reinterpret_cast<f32x4*>(tl + c * 16 + 4 * (g ^ sw)) =
            f32x4{(float)ll[0], (float)ll[1], (float)ll[2], (float)ll[3]};
        *reinterpret_cast<f32x4*>(tl + c * 16 + 4 * ((2 + g) ^ sw)) =
            f32x4{(float)ll[4], (float)ll[5], (float)ll[6], (float)ll[7]};
        float* dst = ljd + (tile * KB + kb) * kLjTile + 16 * H;
#pragma unroll
        for (int u = 0; u < 2; ++u) {
          const int rr = 16 * u + (lane >> 2), pc = lane & 3;
          *reinterpret_cast<f32x4*>(dst + rr * 32 + 4 * pc) =
              *reinterpret_cast<const f32x4*>(tl + rr * 16 + 4 * (pc ^ ljd_swz(rr)));
        }
      }
      // Sparse stored log-joint (fgmm_common.hpp): this wave's 16 components of each
      // row (register groups 2H, 2H + 1), with their max in its half of the maxima.
      if constexpr (LJ)
        lj_put_rows_g<2>(lj + (tile * KB + kb) * kLjTile, ljmax + ((tile * KB + kb) * 2 + H) * 32, c, g,
                         2 * H, ll, bm, acc, run_max, dense != 0);
      if constexpr (LJM == kLjmNeed) {
        const float R = lj_row_max(bm);   // the row's maximum over this wave's 16 components
        if (rexact) {
          if (g == 0) rmax_l[(wave * KB + kb) * 32 + c] = bf16_bits_up(R);
        } else {
          // As the isotropic pass 1: a half block kLjSkipGap below the half's running
          // max cannot carry a nonzero responsibility (logZ2 is above both halves' maxima).
          run_max = fmaxf(run_max, R);
          const bool nb = valid && (dense != 0 || !(R - run_max < -kLjSkipGap));
          const unsigned bits = (unsigned)__builtin_amdgcn_ballot_w64(nb);
          if (lane == 0) ljmask[(tile * KB + kb) * 2 + H] = bits;
        }
      }
      if (MB == 1) lds_barrier();
    };
    for (int kb = 0; kb < KB; kb += 2) {
      step(kb, std::integral_constant<int, 0>{});
      if (kb + 1 >= KB) break;
      step(kb + 1, std::integral_constant<int, 1>{});
    }
  };
  if (h == 0) {
    run(std::integral_constant<int, 0>{});
  } else {
    run(std::integral_constant<int, 1>{});
  }

  // Merge the four partial (max, sum) pairs of a row: the lane-halves first, then
  // the second wave's pair through LDS, in a fixed order.
  double m1 = fmax(mx, __shfl_xor(mx, 32));
  {
    const double mo = __shfl_xor(mx, 32);
    const float so = __shfl_xor(sm, 32);
    const double ms = (m1 == -INFINITY) ? 0.0 : m1;
    sm = sm * fast_exp2((float)(mx - ms)) + so * fast_exp2((float)(mo - ms));
  }
  double* px = reinterpret_cast<double*>(ex);                 // [2][kWaves][64] max, then sum
  float* ps = reinterpret_cast<float*>(px + 2 * kWaves * 64);
  lds_barrier();   // every wave has read its last exchange slot
  px[(h * kWaves + rg) * 64 + lane] = m1;
  ps[(h * kWaves + rg) * 64 + lane] = sm;
  lds_barrier();
  // Both waves form logZ2 from the same two pairs (max and sum commute, so the
  // result is the same bits in each).
  const double mo = px[((1 - h) * kWaves + rg) * 64 + lane];
  const float so = ps[((1 - h) * kWaves + rg) * 64 + lane];
  const double mn = fmax(m1, mo);
  const double ms = (mn == -INFINITY) ? 0.0 : mn;
  const float tot = sm * fast_exp2((float)(m1 - ms)) + so * fast_exp2((float)(mo - ms));
  const double lz2 = mn + (double)log2f(tot);
  if (h == 0 && valid && g == 0) {
    rowstat[row] = lz2;
    if (logZ) logZ[row] = (float)(lz2 * kLn2);
  }
  if constexpr (ST) {
    // The three bf16 parts of this wave's chunks of the row's features (row-major,
    // ljd_rs(DP) apart, chunk q at columns 16 q .. 16 q + 15 as pass 1 orders them)
    // and, from one wave, the row's logZ2 as a (hi, lo) float pair; +inf for a row
    // past N, whose responsibilities are then exactly 0.
    constexpr int RS = ljd_rs(DP);
    __bf16* xp = xsplit + tile * (3 * 32 * RS) + c * RS + 8 * g;
#pragma unroll
    for (int qq = 0; qq < NQH; ++qq) {
#pragma unroll
      for (int t = 0; t < 3; ++t)
        *reinterpret_cast<bf16x8*>(xp + t * 32 * RS + 16 * (h * NQH + qq)) = xb[qq][t];
    }
    if (h == 0 && g == 0) {
      const float zh = valid ? (float)lz2 : INFINITY;
      const float zl = (valid && lz2 > -INFINITY && lz2 < INFINITY) ? (float)(lz2 - (double)zh) : 0.0f;
      zpair[tile * 32 + c] = make_float2(zh, zl);
    }
  }
  // Each wave's need masks from its own maxima; pass 2 ORs the two words.
  if constexpr (LJ) {
    if (g == 0)
      lj_put_masks(ljmax + tile * KB * 64 + h * 32, ljmask + tile * KB * 2 + h, ljcount + (tile & 63), KB, c,
                   lz2, valid, dense != 0, 64, 2);
  }
  if constexpr (LJM == kLjmNeed) {
    if (rexact) {
      const unsigned short* rm = rmax_l + wave * KB * 32 + c;
      if (g == 0)
        need_put_masks([&](int kb) { return bf16_bits_to_float(rm[kb * 32]); }, ljmask + tile * KB * 2 + h,
                       nullptr, KB, c, lz2, valid, dense != 0, 2);
    } else {
      // A row whose logZ2 is NaN gets its bit in every block, as the exact test gives it.
      const unsigned nanbits = (unsigned)__builtin_amdgcn_ballot_w64(valid && g == 0 && lz2 != lz2);
      if (lane == 0 && nanbits != 0)
        for (int kb = 0; kb < KB; ++kb) ljmask[(tile * KB + kb) * 2 + h] |= nanbits;
    }
  }
}

// ---------------------------------------------------------------------------
// The probe of FGMM_FLAG_STORE_LOGJOINT_AUTO: one workgroup per sampled 32-row tile;
// its waves take the component blocks in turn and form each row's block maximum R
// of the log-joint in LDS.  An estimate suffices here, so the contraction keeps two
// of pass 1's seven steps per 16-feature chunk (the centring step and x1 w1), each
// row's chunks whole in one wave.  Then, per row, the blocks with R >= M -
// kLjNeedGap (M the row's largest R) are counted: an estimate of the pairs pass 1
// will mark as needed, since logZ2 >= M.  The tile's count is written; the kernels
// that need the choice sum the counts themselves (probe_selects).
// ---------------------------------------------------------------------------
constexpr int kProbeWaves = 16;
template <int DP>
__global__ __launch_bounds__(64 * kProbeWaves) void diag_store_probe(const float* __restrict__ X, int64_t ldx,
                                                                     int64_t N, int D,
                                                                     const bf16x8* __restrict__ mu3,
                                                                     const double* __restrict__ kc_x6, int KB,
                                                                     int ntile, unsigned* __restrict__ count) {
  constexpr int NQ = DP / 8;
  __shared__ float rmax[kProbeMaxKB * 32];
  __shared__ unsigned part[kProbeWaves];
  const int s = blockIdx.x;
  const int tid = threadIdx.x, lane = tid & 63;
  const int wave = __builtin_amdgcn_readfirstlane(tid >> 6);
  const int c = lane & 31, g = lane >> 5;
  const int64_t tile = probe_tile(s, N, ntile);
  const int64_t row = tile * 32 + c;
  const bool valid = row < N;

  bf16x8 xh[NQ];
#pragma unroll
  for (int q = 0; q < NQ; ++q) {
    const f32x4 x = load_row4(X, ldx, row, 8 * q + 4 * g, D, valid);
    xh[q] = to_bf16x8(x * x, x);
  }
  const bf16x8 ones = x6c_ones(lane);
  for (int kb = wave; kb < KB; kb += kProbeWaves) {
    const bf16x8* mp = mu3 + (int64_t)kb * NQ * 4 * 64 + lane;
    bf16x8 a0[NQ], a3[NQ];
#pragma unroll
    for (int q = 0; q < NQ; ++q) {
      a0[q] = mp[(q * 4 + 0) * 64];
      a3[q] = mp[(q * 4 + 3) * 64];
    }
    f32x16 acc[4] = {zero16(), zero16(), zero16(), zero16()};
#pragma unroll
    for (int q = 0; q < NQ; ++q) {
      acc[q & 3] = mfma_bf16(a3[q], ones, acc[q & 3]);
      acc[q & 3] = mfma_bf16(a0[q], xh[q], acc[q & 3]);
    }
    const double* kp = kc_x6 + (int64_t)kb * 32 + g * 16;
    double bm = -INFINITY;
#pragma unroll
    for (int i = 0; i < 16; ++i) {
      const float xm = (acc[0][i] + acc[1][i]) + (acc[2][i] + acc[3][i]);
      bm = fmax(bm, kp[i] + (double)xm);
    }
    const float R = lj_row_max(bm);
    if (g == 0) rmax[kb * 32 + c] = R;
  }
  __syncthreads();
  // Row c's maximum and needed blocks; the waves split the blocks again.
  unsigned need = 0;
  if (g == 0 && valid) {
    float M = -INFINITY;
    for (int kb = 0; kb < KB; ++kb) M = fmaxf(M, rmax[kb * 32 + c]);
    for (int kb = wave; kb < KB; kb += kProbeWaves) need += (rmax[kb * 32 + c] - M >= -kLjNeedGap) ? 1u : 0u;
  }
#pragma unroll
  for (int o = 32; o > 0; o >>= 1) need += __shfl_xor(need, o);
  if (lane == 0) part[wave] = need;
  __syncthreads();
  if (tid == 0) {
    unsigned tot = 0;
    for (int w = 0; w < kProbeWaves; ++w) tot += part[w];
    count[s] = tot;
  }
}

// ---------------------------------------------------------------------------
// Pass 1 above D = 128 (any D): the component-tiled form of the isotropic
// iso_lse_ctile over the diagonal features.  Each wave owns a 32-row tile; per
// component tile of CTB blocks (ctile_blocks) it streams its rows' chunks of 8 dimensions
// from global memory (lane-half g: dimensions 8q + 4g .. + 3 as [x^2, x], split three
// ways into bf16) against the tile's [-w, 2v] operands and centring offsets, which
// the four waves share through an LDS double buffer of two-chunk stages.  Chunk q
// accumulates into chain q % 4 (x6c_tile's products and order); the chains are
// added as ((c0 + c1) + c2) + c3 and ll2 = C'_k + S in fp64.  Need bounds per half
// block (16 components) as diag_lse_x6 leaves them.  With LJM = kLjmStore (the
// stored plan, D up to 256) the log-joint is written in the register-order tiles
// that diag_accum_lj reads.
// ---------------------------------------------------------------------------
template <int LJM, int CTB>
__global__ __attribute__((amdgpu_flat_work_group_size(64 * kCtWaves, 64 * kCtWaves),
                          amdgpu_waves_per_eu(CTB == 2 ? 2 : 1, CTB == 2 ? 2 : 1)))
void diag_lse_ctile(const float* __restrict__ X, int64_t ldx, int64_t N, int D, int NQ,
                    const bf16x8* __restrict__ mu3, const double* __restrict__ kc_x6, int KB,
                    float* __restrict__ logZ, double* __restrict__ rowstat, float* __restrict__ lj,
                    uint2* __restrict__ ljmask, int dense, int rexact) {
  constexpr bool LJ = LJM == kLjmStore;
  constexpr int NT = 64 * kCtWaves;
  constexpr int SO = ctile_stage_ops(CTB);   // bf16x8 per two-chunk operand stage
  constexpr int LPT = SO / NT;               // operand loads per thread per stage
  static_assert(SO % NT == 0 && CTB * 32 <= NT, "stage split");

  extern __shared__ __align__(16) unsigned char lds_raw[];
  bf16x8* mu_l = reinterpret_cast<bf16x8*>(lds_raw);                                       // [2][stage]
  double* kc_l = reinterpret_cast<double*>(lds_raw + 2 * SO * sizeof(bf16x8));   // [2][blocks*32]
  unsigned short* rmax_l = reinterpret_cast<unsigned short*>(lds_raw + lse_ctile_base(CTB));  // [wave][KB][2][32]

  const int tid = threadIdx.x, lane = tid & 63;
  const int wave = __builtin_amdgcn_readfirstlane(tid >> 6);
  const int c = lane & 31, g = lane >> 5;
  const int64_t tile = (int64_t)blockIdx.x * kCtWaves + wave;   // 32-row tile
  const int64_t row = tile * 32 + c;
  const bool valid = row < N;
  const int NS = NQ / 2;                        // stages per component tile (even: NQ % 4 == 0)
  const int nstage = (int)cdiv(KB, CTB) * NS;
  const int nq_full = D / 8;                    // chunks that end at or before D

  // Operand stages exactly as iso_lse_ctile: thread element u covers block u / 2 of
  // the tile, entry (u % 2) * NT + tid of its 512; blocks past KB read zero.
  const int64_t blk_ops = (int64_t)NQ * 4 * 64;
  const int64_t all_ops = (int64_t)KB * blk_ops;
  bf16x8 st[LPT];
  double kst = -INFINITY;
  auto fetch = [&](int s) __attribute__((always_inline)) {
    const int ct = s / NS, sp = s - ct * NS;
    const int64_t base = (int64_t)ct * CTB * blk_ops + (int64_t)sp * 2 * 4 * 64;
    int64_t avail = (all_ops - base) * (int64_t)sizeof(bf16x8);
    if (avail > ((int64_t)1 << 31) - 16) avail = ((int64_t)1 << 31) - 16;
    const buf_rsrc r = make_rsrc(mu3 + base, (uint32_t)avail);
#pragma unroll
    for (int u = 0; u < LPT; ++u) {
      const int soff = (int)(((int64_t)(u >> 1) * blk_ops + (u & 1) * NT) * (int64_t)sizeof(bf16x8));
      st[u] = __builtin_bit_cast(bf16x8, __builtin_amdgcn_raw_buffer_load_b128(r, tid * (int)sizeof(bf16x8), soff, 0));
    }
    if (sp == 0 && tid < CTB * 32) {
      const int64_t kc = (int64_t)ct * CTB * 32 + tid;
      kst = kc < (int64_t)KB * 32 ? kc_x6[kc] : -INFINITY;
    }
  };
  auto commit = [&](int s, int buf) __attribute__((always_inline)) {
    const int ct = s / NS, sp = s - ct * NS;
#pragma unroll
    for (int u = 0; u < LPT; ++u) mu_l[buf * SO + u * NT + tid] = st[u];
    if (sp == 0 && tid < CTB * 32) kc_l[(ct & 1) * CTB * 32 + tid] = kst;
  };

  // The wave's rows, dimensions 8q + 4g .. + 3 of chunk q (zero past D and N).
  const float* xrow = X + (valid ? row : 0) * ldx + 4 * g;
  auto xload = [&](int q) __attribute__((always_inline)) -> f32x4 {
    if (q < nq_full) {
      const f32x4 v = *reinterpret_cast<const f32x4*>(xrow + 8 * q);
      return valid ? v : zero4();
    }
    return load_row4(X, ldx, row, 8 * q + 4 * g, D, valid);
  };
  f32x4 xr[2][2];   // [stage parity][chunk in the pair]
  auto xstage = [&](int s, f32x4 (&dst)[2]) __attribute__((always_inline)) {
    if (s >= nstage) return;
    const int sp = s % NS;
    dst[0] = xload(2 * sp);
    dst[1] = xload(2 * sp + 1);
  };

  fetch(0);
  xstage(0, xr[0]);
  commit(0, 0);
  lds_barrier();

  f32x16 acc[CTB][kCtChains];
#pragma unroll
  for (int b = 0; b < CTB; ++b) {
#pragma unroll
    for (int h = 0; h < kCtChains; ++h) acc[b][h] = zero16();
  }
  const bf16x8 ones = x6c_ones(lane);
  double mx = -INFINITY;
  float sm = 0.0f;
  float run_max = -INFINITY;   // running max of the row's half-block maxima (running-max bound)

  // Component tile ct is complete: log-joint, log-sum-exp and need bounds per block.
  auto finish_tile = [&](int ct) __attribute__((always_inline)) {
    const double* kp0 = kc_l + (ct & 1) * CTB * 32 + g * 16;
#pragma unroll
    for (int b = 0; b < CTB; ++b) {
      const int kb = ct * CTB + b;
      if (kb < KB) {
        double ll[16];
        double bh[2] = {-INFINITY, -INFINITY};   // maxima of the half blocks (registers 0-7, 8-15)
#pragma unroll
        for (int i = 0; i < 16; ++i) {
          const float S = ((acc[b][0][i] + acc[b][1][i]) + acc[b][2][i]) + acc[b][3][i];
          ll[i] = kp0[b * 32 + i] + (double)S;
          bh[i >> 3] = fmax(bh[i >> 3], ll[i]);
        }
        double bm = fmax(bh[0], bh[1]);
        asm volatile("" : "+v"(bm));
        const double mn = fmax(mx, bm);
        const double ms = (mn == -INFINITY) ? 0.0 : mn;
        float a = sm * fast_exp2((float)(mx - ms));
#pragma unroll
        for (int i = 0; i < 16; ++i) a += fast_exp2((float)(ll[i] - ms));
        sm = a;
        mx = mn;
        if constexpr (LJ) {
          lj_store(lj + (tile * KB + kb) * kLjTile, lane, ll);
        } else {
#pragma unroll
          for (int H = 0; H < 2; ++H) {
            const float R = lj_row_max(bh[H]);
            if (rexact) {
              if (g == 0) rmax_l[((wave * KB + kb) * 2 + H) * 32 + c] = bf16_bits_up(R);
            } else {
              run_max = fmaxf(run_max, R);
              const bool nb = valid && (dense != 0 || !(R - run_max < -kLjSkipGap));
              const unsigned bits = (unsigned)__builtin_amdgcn_ballot_w64(nb);
              if (lane == 0) reinterpret_cast<unsigned*>(ljmask)[(tile * KB + kb) * 2 + H] = bits;
            }
          }
        }
      }
#pragma unroll
      for (int h = 0; h < kCtChains; ++h) acc[b][h] = zero16();
    }
  };

  // One stage; P = s & 1 is the LDS buffer and the register stage, the chunks go to
  // chains 2P and 2P + 1 (NS is even).
  auto stage = [&](int ct, int sp, auto par) __attribute__((always_inline)) {
    constexpr int P = decltype(par)::value;
    const int s = ct * NS + sp;
    const bool more = s + 1 < nstage;
    if (more) fetch(s + 1);
    xstage(s + 1, xr[1 - P]);
    const bf16x8* mp = mu_l + P * SO + lane;
    bf16x8 xb[2][3];
#pragma unroll
    for (int qq = 0; qq < 2; ++qq) split3_bf16(xr[P][qq] * xr[P][qq], xr[P][qq], xb[qq]);
#pragma unroll
    for (int b = 0; b < CTB; ++b) {
      bf16x8 a[2][4];
#pragma unroll
      for (int qq = 0; qq < 2; ++qq) {
#pragma unroll
        for (int t = 0; t < 4; ++t) a[qq][t] = mp[b * 512 + (qq * 4 + t) * 64];
      }
      // Steps in x6c_tile's order: x2 mu2, x1 mu3, x3 mu1, x2 mu1, x1 mu2, -o, x1 mu1.
#pragma unroll
      for (int step = 0; step < 7; ++step) {
#pragma unroll
        for (int qq = 0; qq < 2; ++qq) {
          const bf16x8 A = step == 0 ? a[qq][1] : step == 1 ? a[qq][2] : step <= 3 ? a[qq][0]
                         : step == 4 ? a[qq][1] : step == 5 ? a[qq][3] : a[qq][0];
          const bf16x8 B = step == 0 ? xb[qq][1] : step == 1 ? xb[qq][0] : step == 2 ? xb[qq][2]
                         : step == 3 ? xb[qq][1] : step == 4 ? xb[qq][0] : step == 5 ? ones : xb[qq][0];
          acc[b][2 * P + qq] = mfma_bf16(A, B, acc[b][2 * P + qq]);
        }
      }
    }
    if (more) commit(s + 1, 1 - P);
    lds_barrier();
  };
  for (int ct = 0; ct * NS < nstage; ++ct) {
    for (int sp = 0; sp < NS; sp += 2) {
      stage(ct, sp, std::integral_constant<int, 0>{});
      stage(ct, sp + 1, std::integral_constant<int, 1>{});
    }
    finish_tile(ct);
  }

  // Merge the two half-waves that hold the same row.
  const double mo = __shfl_xor(mx, 32);
  const float so = __shfl_xor(sm, 32);
  const double mn = fmax(mx, mo);
  const double ms = (mn == -INFINITY) ? 0.0 : mn;
  const float tot = sm * fast_exp2((float)(mx - ms)) + so * fast_exp2((float)(mo - ms));
  const double lz2 = mn + (double)log2f(tot);
  if (valid && g == 0) {
    rowstat[row] = lz2;
    if (logZ) logZ[row] = (float)(lz2 * kLn2);
  }
  if constexpr (!LJ) {
    unsigned* mk = reinterpret_cast<unsigned*>(ljmask);
    if (rexact) {
#pragma unroll
      for (int H = 0; H < 2; ++H) {
        const unsigned short* rm = rmax_l + (wave * KB * 2 + H) * 32 + c;
        if (g == 0)
          need_put_masks([&](int kb) { return bf16_bits_to_float(rm[kb * 64]); }, mk + tile * KB * 2 + H,
                         nullptr, KB, c, lz2, valid, dense != 0, 2);
      }
    } else {
      // A row whose logZ2 is NaN gets its bit in every half block, as the exact test gives it.
      const unsigned nanbits = (unsigned)__builtin_amdgcn_ballot_w64(valid && g == 0 && lz2 != lz2);
      if (lane == 0 && nanbits != 0)
        for (int kb = 0; kb < KB; ++kb) {
          mk[(tile * KB + kb) * 2] |= nanbits;
          mk[(tile * KB + kb) * 2 + 1] |= nanbits;
        }
    }
  }
}

// ---------------------------------------------------------------------------
// Pass 2 from the sparse stored log-joint (up to D = 128, D a multiple of 32), for
// sparse need masks: as iso_accum_sparse (fgmm_iso.hip), one wave per (row slab, row
// group, component block) fetching only the needed register-row pairs of each tile,
// here accumulating r^T x and r^T x^2.  The same split and order as diag_accum_lj2,
// so the two write the same partials; the needed-pair count of pass 1 picks one.
// ---------------------------------------------------------------------------
constexpr int kSparseSlots = 3;
constexpr int kSparseDepth = 4;
constexpr int kSparseBatch = 256;
constexpr int kSparseWaves = 4;

// Total of the 64 needed-pair counters (one wave, uniform result).
__device__ __forceinline__ unsigned lj_pair_total(const unsigned* __restrict__ count) {
  unsigned v = count[threadIdx.x & 63];
#pragma unroll
  for (int o = 32; o > 0; o >>= 1) v += __shfl_xor(v, o);
  return __builtin_amdgcn_readfirstlane(v);
}

template <int DP>
__global__ __launch_bounds__(64 * kSparseWaves)
void diag_accum_sparse(const float* __restrict__ X, int64_t ldx, int64_t N, const float* __restrict__ lj,
                       const uint2* __restrict__ ljmask, const unsigned* __restrict__ ljcount,
                       int64_t sparse_max, int KB, int KP, const double* __restrict__ rowstat, int nslab,
                       int RG, int64_t rows_per_slab, float* __restrict__ part_mu,
                       float* __restrict__ part_sq, float* __restrict__ part_nk, int dense) {
  constexpr int NJ = DP / 32;
  constexpr int S = kSparseSlots;
  constexpr int PD = kSparseDepth;
  constexpr int BT = kSparseBatch;
  typedef float fNJ __attribute__((ext_vector_type(NJ)));
  __shared__ uint2 work[kSparseWaves][BT];      // the tile's two mask words
  __shared__ unsigned wtile[kSparseWaves][BT];  // and its index in the batch

  if ((int64_t)lj_pair_total(ljcount) > sparse_max) return;
  const int lane = threadIdx.x & 63;
  const int wave = __builtin_amdgcn_readfirstlane(threadIdx.x >> 6);
  const int c = lane & 31, g = lane >> 5;
  const int64_t w = (int64_t)blockIdx.x * kSparseWaves + wave;
  if (w >= (int64_t)nslab * RG * KB) return;
  const int kb = (int)(w % KB);
  const int rg = (int)((w / KB) % RG);
  const int slab = (int)(w / ((int64_t)KB * RG));
  const int TR = 32 * RG;

  const int64_t r_begin = (int64_t)slab * rows_per_slab;
  int64_t r_end = r_begin + rows_per_slab;
  if (r_end > N) r_end = N;
  const int ntiles = r_end > r_begin ? (int)cdiv(r_end - r_begin, TR) : 0;

  f32x16 accx[NJ], accq[NJ];
#pragma unroll
  for (int j = 0; j < NJ; ++j) {
    accx[j] = zero16();
    accq[j] = zero16();
  }
  float nk = 0.0f;

  const int64_t row00 = r_begin + rg * 32;
  const float* lj0 = lj + ((row00 >> 5) * KB + kb) * kLjTile;
  const double* rs0 = rowstat + row00;
  const float* x0 = X + row00 * ldx;
  const int64_t lj_step = (int64_t)RG * KB * kLjTile, x_step = TR * ldx;
  auto windows = [&](int t, buf_rsrc& lr, buf_rsrc& rr, buf_rsrc& xr) {
    lr = make_rsrc(lj0 + t * lj_step, kLjTile * 4);
    rr = make_rsrc(rs0 + (int64_t)t * TR, 32 * sizeof(double));
    xr = make_rsrc(x0 + t * x_step, (uint32_t)(32 * ldx * 4));
  };

  float sl[PD][S];
  double sz[PD][S];
  fNJ sx[PD][S];
  unsigned smk[PD];   // rows needed by either half of the block (uniform)
  unsigned smh[PD];   // rows needed by this lane's half (components 16 (c >> 4) ..)
  int stl[PD];

  // Each half of a row's line is stored by its own pass-1 wave, which may leave it
  // out (it is then negligible and its mask bit clear), so a lane reads its
  // component's value (and the row's logZ2) under its half's mask word mh.  Its X
  // columns feed every component of the block: they follow the row mask m.
  auto load_pair = [&](const buf_rsrc& lr, const buf_rsrc& rr, const buf_rsrc& xr, unsigned m, unsigned mh,
                       int ro, bool used, float& l, double& z, fNJ& x) {
    const int row = ro + 4 * g;
    const bool need = used && ((mh >> row) & 1u);
    const bool row_need = used && ((m >> row) & 1u);
    l = buf_load_f32<kBufNt>(lr, buf_off(need ? (row * 32 + c) * 4 : kBufOob));
    z = buf_load_f64(rr, buf_off(need ? row * (int)sizeof(double) : kBufOob));
    const int xo = buf_off(row_need ? (int)((row * ldx + NJ * c) * 4) : kBufOob);
    if constexpr (NJ == 4) {
      x = buf_load_f32x4(xr, xo);
    } else if constexpr (NJ == 3) {
      x = __builtin_bit_cast(fNJ, __builtin_amdgcn_raw_buffer_load_b96(xr, xo, 0, 0));
    } else if constexpr (NJ == 2) {
      x = __builtin_bit_cast(fNJ, __builtin_amdgcn_raw_buffer_load_b64(xr, xo, 0, 0));
    } else {
      x = __builtin_bit_cast(fNJ, __builtin_amdgcn_raw_buffer_load_b32(xr, xo, 0, 0));
    }
  };
  // One pair's contribution, in the arithmetic of diag_accum_lj2.
  auto accumulate = [&](unsigned mh, int ro, float l, double q, const fNJ& x) {
    const bool need = (mh >> (ro + 4 * g)) & 1u;
    const float zh = (float)q;
    const float zl = (q > -INFINITY && q < INFINITY) ? (float)(q - (double)zh) : 0.0f;
    const float rv = need ? fast_exp2((l - zh) - zl) : 0.0f;
    nk += rv;
    if (dense || __builtin_amdgcn_ballot_w64(rv != 0.0f) != 0) {
#pragma unroll
      for (int jj = 0; jj < NJ; ++jj) {
        accx[jj] = mfma32(rv, x[jj], accx[jj]);
        accq[jj] = mfma32(rv, x[jj] * x[jj], accq[jj]);
      }
    }
  };
  auto issue = [&](int k, int cnt, int b0, int u) {
    unsigned m = 0u, mh = 0u;
    int t = 0;
    if (k < cnt) {
      const uint2 e = work[wave][k];
      const unsigned mx = __builtin_amdgcn_readfirstlane(e.x), my = __builtin_amdgcn_readfirstlane(e.y);
      m = mx | my;
      mh = c < 16 ? mx : my;
      t = b0 + __builtin_amdgcn_readfirstlane(wtile[wave][k]);
    }
    smk[u] = m;
    smh[u] = mh;
    stl[u] = t;
    buf_rsrc lr, rr, xr;
    windows(t, lr, rr, xr);
    unsigned pm = lj_pair_mask(m);
#pragma unroll
    for (int j = 0; j < S; ++j) {
      const bool used = pm != 0u;
      const int ro = used ? __builtin_ctz(pm) : 0;
      pm &= pm - 1u;
      load_pair(lr, rr, xr, m, mh, ro, used, sl[u][j], sz[u][j], sx[u][j]);
    }
  };
  auto process = [&](int u) {
    const unsigned m = smk[u], mh = smh[u];
    if (m == 0u) return;
    unsigned pm = lj_pair_mask(m);
#pragma unroll
    for (int j = 0; j < S; ++j) {
      if (pm == 0u) return;
      const int ro = __builtin_ctz(pm);
      pm &= pm - 1u;
      accumulate(mh, ro, sl[u][j], sz[u][j], sx[u][j]);
    }
    if (pm == 0u) return;
    buf_rsrc lr, rr, xr;   // more pairs than slots: load them now
    windows(stl[u], lr, rr, xr);
    while (pm != 0u) {
      const int ro = __builtin_ctz(pm);
      pm &= pm - 1u;
      float l;
      double q;
      fNJ x;
      load_pair(lr, rr, xr, m, mh, ro, true, l, q, x);
      accumulate(mh, ro, l, q, x);
    }
  };

  for (int b0 = 0; b0 < ntiles; b0 += BT) {
    int cnt = 0;
#pragma unroll
    for (int q = 0; q < BT / 64; ++q) {
      const int t = b0 + 64 * q + lane;
      const int64_t row0 = r_begin + (int64_t)t * TR + rg * 32;
      uint2 mm = make_uint2(0u, 0u);
      if (t < ntiles && row0 < r_end) mm = ljmask[(row0 >> 5) * KB + kb];
      const bool any = (mm.x | mm.y) != 0u;
      const unsigned long long bal = __builtin_amdgcn_ballot_w64(any);
      const int pos = cnt + (int)__builtin_amdgcn_mbcnt_hi((unsigned)(bal >> 32),
                                                           __builtin_amdgcn_mbcnt_lo((unsigned)bal, 0u));
      if (any) {
        work[wave][pos] = mm;
        wtile[wave][pos] = (unsigned)(64 * q + lane);
      }
      cnt += __builtin_popcountll(bal);
    }
#pragma unroll
    for (int u = 0; u < PD; ++u) issue(u, cnt, b0, u);
    for (int kk = 0; kk < cnt; kk += PD) {
#pragma unroll
      for (int u = 0; u < PD; ++u) {
        process(u);
        issue(kk + u + PD, cnt, b0, u);
      }
    }
  }

  nk += __shfl_xor(nk, 32);
  const int64_t kbase = ((int64_t)slab * RG + rg) * KP + (int64_t)kb * 32;
#pragma unroll
  for (int i = 0; i < 16; ++i) {
    const int64_t o = (kbase + acc_row(i, g)) * DP + NJ * c;
#pragma unroll
    for (int jj = 0; jj < NJ; ++jj) {
      part_mu[o + jj] = accx[jj][i];
      part_sq[o + jj] = accq[jj][i];
    }
  }
  if (g == 0) part_nk[kbase + c] = nk;
}

// ---------------------------------------------------------------------------
// Pass 2 from the sparse stored log-joint (up to D = 128), for dense need masks (and
// every FGMM_FLAG_DENSE run): the structure of iso_accum_lj (fgmm_iso.hip).  X
// super-tiles, with their rows' logZ2 and the masks of the next tile, are staged in
// LDS for 8 component blocks through two register stages (loop unrolled by two);
// each wave reads the needed log-joint rows of its block one tile ahead with
// range-checked buffer loads and accumulates r^T x and r^T x^2 for the needed
// register-row pairs, in ascending order (unrolled for tiles with 8 or more pairs).
// ---------------------------------------------------------------------------
template <int DP, int CB, int NH>
constexpr size_t accum_lj2_lds_bytes() {
  return (size_t)2 * 32 * (kAccWaves / (CB * NH)) * ((DP + 4) * sizeof(float) + sizeof(float2)) +
         (size_t)2 * kAccWaves * sizeof(uint2);
}

template <int DP, int CB, int NH>
__global__ __attribute__((amdgpu_flat_work_group_size(kAccThreads, kAccThreads), amdgpu_waves_per_eu(2, 2)))
void diag_accum_lj2(const float* __restrict__ X, int64_t ldx, int64_t N, int D, const float* __restrict__ lj,
                    const uint2* __restrict__ ljmask, const unsigned* __restrict__ ljcount,
                    int64_t sparse_max, int KB, int KP, const double* __restrict__ rowstat, int nslab,
                    int64_t rows_per_slab, float* __restrict__ part_mu, float* __restrict__ part_sq,
                    float* __restrict__ part_nk, int dense) {
  constexpr int NJ = DP / 32 / NH;               // 32-column tiles per wave (each for x and x^2)
  constexpr int RS = DP + 4;
  constexpr int V4 = DP / 4;
  constexpr int RG = kAccWaves / (CB * NH);      // row groups (32 rows each)
  constexpr int TR = 32 * RG;                    // rows per super-tile
  constexpr int NV = TR * V4;                    // float4 per super-tile
  constexpr int LPT = (NV + kAccThreads - 1) / kAccThreads;
  constexpr int NB = 2;                          // register stages
  static_assert(kAccWaves % (CB * NH) == 0 && (DP / 32) % NH == 0, "even split");
  static_assert(TR + kAccWaves <= kAccThreads, "row-state and mask threads");

  // diag_accum_sparse takes the call when pass 1 found the masks sparse.
  if (sparse_max >= 0 && (int64_t)lj_pair_total(ljcount) <= sparse_max) return;

  extern __shared__ __align__(16) unsigned char lds_raw[];
  float* xs = reinterpret_cast<float*>(lds_raw);                                  // [2][TR*RS]
  float2* rz = reinterpret_cast<float2*>(lds_raw + 2 * TR * RS * sizeof(float));  // [2][TR]
  uint2* mk = reinterpret_cast<uint2*>(rz + 2 * TR);                              // [2][kAccWaves]

  const int tid = threadIdx.x, lane = tid & 63;
  const int wave = __builtin_amdgcn_readfirstlane(tid >> 6);
  const int c = lane & 31, g = lane >> 5;
  const int cbw = wave % CB, h = (wave / CB) % NH, rg = wave / (CB * NH);
  const int slab = blockIdx.x % nslab;
  const int cg = blockIdx.x / nslab;
  const int kb = cg * CB + cbw;
  const bool active = kb < KB;
  const int col0 = h * (DP / NH);

  const int64_t r_begin = (int64_t)slab * rows_per_slab;
  int64_t r_end = r_begin + rows_per_slab;
  if (r_end > N) r_end = N;
  const int ntiles = r_end > r_begin ? (int)cdiv(r_end - r_begin, TR) : 0;

  f32x16 accx[NJ], accq[NJ];
#pragma unroll
  for (int j = 0; j < NJ; ++j) {
    accx[j] = zero16();
    accq[j] = zero16();
  }
  float nk = 0.0f;

  // Need masks of (row tile, block): one word per half of the block's components,
  // each from the pass-1 wave that stored that half of the rows' lines (and may
  // have left it out; it is then negligible and its bit clear).  A register-row
  // pair is visited when either half needs a row; a lane reads its value only
  // under its own half's word.
  const buf_rsrc mask_r = make_rsrc(ljmask, (uint32_t)(cdiv(N, 32) * KB * sizeof(uint2)));
  auto mask_off = [&](int t, int rgw, int kbw) -> int {
    const int64_t row0 = r_begin + (int64_t)t * TR + rgw * 32;
    return (t < ntiles && row0 < r_end && kbw < KB) ? (int)(((row0 >> 5) * KB + kbw) * sizeof(uint2)) : kBufOob;
  };
  auto mask_load = [&](int off) -> uint2 {
    const auto v = __builtin_amdgcn_raw_buffer_load_b64(mask_r, buf_off(off), 0, 0);
    return make_uint2(v[0], v[1]);
  };

  const bool ragged = (D & 3) != 0;
  auto fetch = [&](int t, f32x4 (&st)[LPT], double& rqv, uint2& mqv) {
    const int64_t row0 = r_begin + (int64_t)t * TR;
    int nrow = 0;
    if (t < ntiles) nrow = (int)(r_end - row0 < TR ? r_end - row0 : TR);
    const buf_rsrc xr = make_rsrc(nrow ? X + row0 * ldx : X, (uint32_t)(nrow * ldx * 4));
#pragma unroll
    for (int q = 0; q < LPT; ++q) {
      const int idx = q * kAccThreads + tid;
      const int r = idx / V4, col = (idx % V4) * 4;
      const bool ok = (NV % kAccThreads == 0 || idx < NV) && r < nrow && col < D;
      st[q] = buf_load_f32x4(xr, buf_off(ok ? (int)((r * ldx + col) * 4) : kBufOob));
    }
    const buf_rsrc rr = make_rsrc(nrow ? rowstat + row0 : rowstat, (uint32_t)(nrow * sizeof(double)));
    const double q2 = buf_load_f64(rr, buf_off(tid < nrow ? tid * (int)sizeof(double) : kBufOob));
    rqv = tid < nrow ? q2 : INFINITY;   // rows past the slab: logZ2 = +inf, hence r = 0
    const int w = tid - TR;
    mqv = mask_load((w >= 0 && w < kAccWaves) ? mask_off(t + NB - 1, w / (CB * NH), cg * CB + w % CB)
                                              : kBufOob);
  };
  auto commit = [&](int buf, const f32x4 (&st)[LPT], double rqv, uint2 mqv) {
    float* dst = xs + buf * TR * RS;
#pragma unroll
    for (int q = 0; q < LPT; ++q) {
      const int idx = q * kAccThreads + tid;
      if (NV % kAccThreads == 0 || idx < NV) {
        const int col = (idx % V4) * 4;
        f32x4 v = st[q];
        if (ragged) {
          if (col + 1 >= D) v.y = 0.0f;
          if (col + 2 >= D) v.z = 0.0f;
          if (col + 3 >= D) v.w = 0.0f;
        }
        *reinterpret_cast<f32x4*>(dst + (idx / V4) * RS + col) = v;
      }
    }
    if (tid < TR) {
      const float hi = (float)rqv;
      const float lo = (rqv > -INFINITY && rqv < INFINITY) ? (float)(rqv - (double)hi) : 0.0f;
      rz[buf * TR + tid] = make_float2(hi, lo);
    }
    if (tid >= TR && tid < TR + kAccWaves) mk[buf * kAccWaves + tid - TR] = mqv;
  };
  auto lj_fetch = [&](int t, uint2 m, f32x16& v) {
    const int64_t row0 = r_begin + (int64_t)t * TR + rg * 32;
    const bool any = (m.x | m.y) != 0u;
    const unsigned mh = c < 16 ? m.x : m.y;
    const buf_rsrc lr = make_rsrc(any ? lj + ((row0 >> 5) * KB + kb) * kLjTile : lj, any ? kLjTile * 4 : 0);
#pragma unroll
    for (int i = 0; i < 16; ++i) {
      const int row = 8 * (i >> 2) + (i & 3) + 4 * g;
      v[i] = buf_load_f32<kBufNt>(lr, buf_off(((mh >> row) & 1u) ? (row * 32 + c) * 4 : kBufOob));
    }
  };
  auto uniform = [](uint2 m) {
    return make_uint2(__builtin_amdgcn_readfirstlane(m.x), __builtin_amdgcn_readfirstlane(m.y));
  };

  f32x4 stg[NB][LPT];
  double rqs[NB];
  uint2 mqs[NB];
  f32x16 ljb[NB];
  uint2 mcur = make_uint2(0u, 0u);   // need masks of the current tile

  // One register-row pair: r for the needed lanes, then the steps of r^T x and r^T x^2.
  auto pair = [&](unsigned mg, int ro, float l, float2 z, const float* xb) {
    const float rv = ((mg >> ro) & 1u) ? fast_exp2((l - z.x) - z.y) : 0.0f;
    if (NH == 1 || h == 0) nk += rv;
    if (dense || __builtin_amdgcn_ballot_w64(rv != 0.0f) != 0) {
#pragma unroll
      for (int jj = 0; jj < NJ; ++jj) {
        const float xv = xb[ro * RS + 32 * jj];
        accx[jj] = mfma32(rv, xv, accx[jj]);
        accq[jj] = mfma32(rv, xv * xv, accq[jj]);
      }
    }
  };

  auto step = [&](int t, auto par) {
    constexpr int P = decltype(par)::value;
    const int lb = t & 1;
    const uint2 ma = uniform(mk[lb * kAccWaves + wave]);   // tile t + 1
    lj_fetch(t + 1, ma, ljb[1 - P]);
    fetch(t + 2, stg[P], rqs[P], mqs[P]);
    const unsigned mc = mcur.x | mcur.y;
    const float* xt = xs + lb * TR * RS + rg * 32 * RS;
    const float2* rt = rz + lb * TR + rg * 32 + 4 * g;
    if (active && mc != 0u) {
      const float* xbase = xt + 4 * g * RS + col0 + c;
      unsigned pm = lj_pair_mask(mc);
      const unsigned mg = (c < 16 ? mcur.x : mcur.y) >> (4 * g);
      // Unrolled for dense tiles where the accumulators leave registers for it.
      if (NJ <= 2 && __builtin_popcount(pm) >= 8) {
#pragma unroll
        for (int q = 0; q < 4; ++q) {
#pragma unroll
          for (int j = 0; j < 4; ++j) {
            const int ro = 8 * q + j;
            if ((pm >> ro) & 1u) pair(mg, ro, ljb[P][4 * q + j], rt[ro], xbase);
          }
        }
      } else {
        while (pm != 0u) {
          const int ro = __builtin_ctz(pm);
          pm &= pm - 1u;
          pair(mg, ro, ljb[P][4 * (ro >> 3) + (ro & 3)], rt[ro], xbase);
        }
      }
    }
    if (t + 1 < ntiles) commit(lb ^ 1, stg[1 - P], rqs[1 - P], mqs[1 - P]);
    lds_barrier();
    mcur = ma;
  };

  if (ntiles > 0) {
    fetch(0, stg[0], rqs[0], mqs[0]);
    fetch(1, stg[1], rqs[1], mqs[1]);
    mcur = uniform(mask_load(mask_off(0, rg, kb)));
    lj_fetch(0, mcur, ljb[0]);
    commit(0, stg[0], rqs[0], mqs[0]);
    lds_barrier();
  }
  for (int t = 0; t < ntiles; t += 2) {
    step(t, std::integral_constant<int, 0>{});
    if (t + 1 >= ntiles) break;
    step(t + 1, std::integral_constant<int, 1>{});
  }

  if (active) {
    nk += __shfl_xor(nk, 32);
    const int64_t kbase = ((int64_t)slab * RG + rg) * KP + (int64_t)kb * 32;
#pragma unroll
    for (int j = 0; j < NJ; ++j) {
#pragma unroll
      for (int i = 0; i < 16; ++i) {
        const int64_t o = (kbase + acc_row(i, g)) * DP + col0 + 32 * j + c;
        part_mu[o] = accx[j][i];
        part_sq[o] = accq[j][i];
      }
    }
    if (g == 0 && h == 0) part_nk[kbase + c] = nk;
  }
}

// ---------------------------------------------------------------------------
// Pass 2 from the stored log-joint: grid over (row slab x group of CB component
// blocks); eight waves = CB component blocks x NH column parts x 8 / (CB NH) row
// groups of 32 rows (NH = 2 above D = 128, or at D = 128 with 4 blocks: one wave's
// accumulators for x and x^2 over all of D would not fit in registers).  Each wave
// reads the log-joint tile of its block and rows (4 KiB), forms
// r = 2^(ll2 - logZ2) and accumulates r^T [x | x^2] for its columns on the matrix
// cores from the X tile that the workgroup's blocks share in LDS.  logZ2 sits in
// LDS as a hi + lo pair of floats, so ll2 - logZ2 keeps the accuracy of the fp32
// log-joint.
// ---------------------------------------------------------------------------
template <int DP, int CB, int NH>
constexpr size_t accum_lj_lds_bytes() {
  return (size_t)2 * 32 * (kAccWaves / (CB * NH)) * ((DP + 4) * sizeof(float) + sizeof(float2));
}

template <int DP, int CB, int NH>
__global__ __attribute__((amdgpu_flat_work_group_size(kAccThreads, kAccThreads), amdgpu_waves_per_eu(2, 2)))
void diag_accum_lj(const float* __restrict__ X, int64_t ldx, int64_t N, int D,
                   const float* __restrict__ lj, int KB, int KP, const double* __restrict__ rowstat,
                   int nslab, int64_t rows_per_slab, float* __restrict__ part_mu,
                   float* __restrict__ part_sq, float* __restrict__ part_nk, int dense) {
  constexpr int NJ = DP / 32 / NH;               // 32-column tiles per wave (each for x and x^2)
  constexpr int RS = DP + 4;
  constexpr int V4 = DP / 4;
  constexpr int RG = kAccWaves / (CB * NH);      // row groups (32 rows each)
  constexpr int TR = 32 * RG;                    // rows per super-tile
  constexpr int NV = TR * V4;                    // float4 per super-tile
  constexpr int LPT = (NV + kAccThreads - 1) / kAccThreads;
  static_assert(kAccWaves % (CB * NH) == 0 && (DP / 32) % NH == 0, "even split");

  extern __shared__ __align__(16) unsigned char lds_raw[];
  float* xs = reinterpret_cast<float*>(lds_raw);                                  // [2][TR*RS]
  float2* rz = reinterpret_cast<float2*>(lds_raw + 2 * TR * RS * sizeof(float));  // [2][TR]

  const int tid = threadIdx.x, lane = tid & 63, wave = tid >> 6;
  const int c = lane & 31, g = lane >> 5;
  const int cbw = wave % CB, h = (wave / CB) % NH, rg = wave / (CB * NH);
  const int slab = blockIdx.x % nslab;
  const int cg = blockIdx.x / nslab;
  const int kb = cg * CB + cbw;
  const bool active = kb < KB;
  const int col0 = h * (DP / NH);

  const int64_t r_begin = (int64_t)slab * rows_per_slab;
  int64_t r_end = r_begin + rows_per_slab;
  if (r_end > N) r_end = N;
  const int ntiles = r_end > r_begin ? (int)cdiv(r_end - r_begin, TR) : 0;

  f32x16 accx[NJ], accq[NJ];
#pragma unroll
  for (int j = 0; j < NJ; ++j) {
    accx[j] = zero16();
    accq[j] = zero16();
  }
  float nk = 0.0f;

  // X tiles and row logZ2 go global -> registers -> LDS through two register
  // stages (tile t + 2 is loaded while tile t is processed; the LDS-only barrier
  // leaves the loads in flight).
  f32x4 stage[LPT], stage2[LPT];
  double rq = INFINITY, rq2 = INFINITY;
  const bool full_d = (D == DP);
  auto fetch = [&](int t, f32x4 (&stage)[LPT], double& rq) {
    const int64_t row0 = r_begin + (int64_t)t * TR;
    if (full_d && row0 + TR <= r_end) {
      const float* src = X + row0 * ldx;
#pragma unroll
      for (int q = 0; q < LPT; ++q) {
        const int idx = q * kAccThreads + tid;
        if (NV % kAccThreads == 0 || idx < NV)
          stage[q] = *reinterpret_cast<const f32x4*>(src + (int64_t)(idx / V4) * ldx + (idx % V4) * 4);
      }
    } else {
#pragma unroll
      for (int q = 0; q < LPT; ++q) {
        const int idx = q * kAccThreads + tid;
        const int64_t row = row0 + idx / V4;
        stage[q] = load_row4(X, ldx, row, (idx % V4) * 4, D, idx < NV && row < r_end);
      }
    }
    if (tid < TR) {
      const int64_t row = row0 + tid;
      rq = (row < r_end) ? rowstat[row] : INFINITY;
    }
  };
  auto commit = [&](int buf, const f32x4 (&stage)[LPT], double rq) {
    float* dst = xs + buf * TR * RS;
#pragma unroll
    for (int q = 0; q < LPT; ++q) {
      const int idx = q * kAccThreads + tid;
      if (NV % kAccThreads == 0 || idx < NV)
        *reinterpret_cast<f32x4*>(dst + (idx / V4) * RS + (idx % V4) * 4) = stage[q];
    }
    if (tid < TR) {
      // Rows past the slab get logZ2 = +inf, hence r = 0.
      const float hi = (float)rq;
      const float lo = (rq > -INFINITY && rq < INFINITY) ? (float)(rq - (double)hi) : 0.0f;
      rz[buf * TR + tid] = make_float2(hi, lo);
    }
  };
  auto lj_fetch = [&](int t, f32x4 (&v)[4]) {
    const int64_t row0 = r_begin + (int64_t)t * TR + rg * 32;
    if (active && row0 < r_end) {
      lj_load(lj + ((row0 >> 5) * KB + kb) * kLjTile, lane, v);
    } else {
#pragma unroll
      for (int q = 0; q < 4; ++q) v[q] = zero4();
    }
  };

  // Log-joint tiles two super-tiles ahead, or one with more than 4 accumulator
  // tiles per wave; above 6 the r of each row is formed just before its steps
  // (registers).
  constexpr int kTiles = 2 * NJ;
  constexpr bool kLj2 = kTiles <= 4;
  constexpr bool kInterleave = kTiles > 6;
  f32x4 ljc[4], ljn[4], ljm[4];
  if (ntiles > 0) {
    fetch(0, stage, rq);
    lj_fetch(0, ljc);
    commit(0, stage, rq);
  }
  if (ntiles > 1) {
    fetch(1, stage, rq);
    if (kLj2) lj_fetch(1, ljn);
  }
  lds_barrier();

  for (int t = 0; t < ntiles; ++t) {
    const int buf = t & 1;
    const bool more = t + 1 < ntiles;
    if (t + 2 < ntiles) {
      fetch(t + 2, stage2, rq2);
      if (kLj2) lj_fetch(t + 2, ljm);
    }
    if (!kLj2 && more) lj_fetch(t + 1, ljn);
    const float* xt = xs + buf * TR * RS + rg * 32 * RS;
    const float2* rt = rz + buf * TR + rg * 32 + 4 * g;
    if (active) {
      const float* xbase = xt + 4 * g * RS + col0 + c;
      float r[16];
#pragma unroll
      for (int i = 0; i < 16; ++i) {
        const int ro = 8 * (i >> 2) + (i & 3);
        const float2 z = rt[ro];
        const float rv = fast_exp2((ljc[i >> 2][i & 3] - z.x) - z.y);
        if (NH == 1 || h == 0) nk += rv;
        r[i] = rv;
        if (kInterleave && (dense || __builtin_amdgcn_ballot_w64(rv != 0.0f) != 0)) {
#pragma unroll
          for (int j = 0; j < NJ; ++j) {
            const float xv = xbase[ro * RS + 32 * j];
            accx[j] = mfma32(rv, xv, accx[j]);
            accq[j] = mfma32(rv, xv * xv, accq[j]);
          }
        }
      }
      if constexpr (!kInterleave) {
#pragma unroll
        for (int i = 0; i < 16; ++i) {
          const int ro = 8 * (i >> 2) + (i & 3);
          if (dense || __builtin_amdgcn_ballot_w64(r[i] != 0.0f) != 0) {
#pragma unroll
            for (int j = 0; j < NJ; ++j) {
              const float xv = xbase[ro * RS + 32 * j];
              accx[j] = mfma32(r[i], xv, accx[j]);
              accq[j] = mfma32(r[i], xv * xv, accq[j]);
            }
          }
        }
      }
    }
    if (more) commit(buf ^ 1, stage, rq);
    lds_barrier();
#pragma unroll
    for (int q = 0; q < LPT; ++q) stage[q] = stage2[q];
    rq = rq2;
#pragma unroll
    for (int q = 0; q < 4; ++q) {
      ljc[q] = ljn[q];
      if (kLj2) ljn[q] = ljm[q];
    }
  }

  if (active) {
    nk += __shfl_xor(nk, 32);
    const int64_t kbase = ((int64_t)slab * RG + rg) * KP + (int64_t)kb * 32;
#pragma unroll
    for (int j = 0; j < NJ; ++j) {
#pragma unroll
      for (int i = 0; i < 16; ++i) {
        const int64_t o = (kbase + acc_row(i, g)) * DP + col0 + 32 * j + c;
        part_mu[o] = accx[j][i];
        part_sq[o] = accq[j][i];
      }
    }
    if (g == 0 && h == 0) part_nk[kbase + c] = nk;
  }
}

__host__ size_t x6_lds_bytes_rt(int DP) {
  switch (DP) {
    case 32: return x6_lds_bytes<32>();
    case 64: return x6_lds_bytes<64>();
    case 96: return x6_lds_bytes<96>();
    case 128: return x6_lds_bytes<128>();
    default: return 160 * 1024;
  }
}

// ---------------------------------------------------------------------------
// Pass 2 of the default plan (D <= 128): the log-joint is recomputed only for the
// (row, component block) pairs whose need bit (either half's word) pass 1 set.
// One wave per (row slab, component block), 4 waves of one block per workgroup on
// consecutive slabs (the isotropic gathering kernel's structure), mu's split
// features and centring offsets of the block in LDS for the four.  Per tile of 32
// queued rows: the rows of X (fp32) go to the wave's LDS tile; S = [x^2, x] . [-w, 2v]^T
// is formed as pass 1 forms it, the two halves' chains (x6c_tile_rows_fn, two chains
// each) added in fp32, so the log-joint C'_k + S equals pass 1's; r = 2^(ll2 - logZ2),
// Nk on the VALU, and r^T [X | X^2] on the bf16 matrix cores with r as the A operand:
// r, x and x^2 split exactly into three bf16 values each and the six products of
// significance at least 2^-16 accumulated smallest first (error near an fp32 step's,
// which the sig identity needs), 16 rows per step (steps whose 16 rows carry no
// responsibility are skipped).  sig follows in
// diag_reduce from the moments.
// ---------------------------------------------------------------------------

// fp32 row stride of the X tiles: rows 8 apart (the two lane-halves of a B operand)
// and the 16-byte row accesses of the contraction fall in distinct banks.
__host__ __device__ constexpr int gather_rs(int DP) { return DP + 4; }

__host__ __device__ constexpr size_t gather_lds_bytes(int DP) {
  return (size_t)(DP / 8) * 4 * 64 * 16                          // mu block (bf16x8 operands)
         + (size_t)kGatherWaves * 32 * gather_rs(DP) * 4          // X tile per wave
         + (size_t)kGatherWaves * 32 * sizeof(double)              // logZ2 per wave
         + (size_t)kGatherWaves * 64 * sizeof(int);                // row queue per wave
}
__host__ __device__ constexpr int gather_groups(int nslab) { return (nslab + kGatherWaves - 1) / kGatherWaves; }
__host__ inline int64_t gather_grid(int nslab, int KB) { return gather_item_grid(gather_groups(nslab), KB); }

// Waves per SIMD of the gathering pass: two where a wave's registers and the
// workgroup's LDS allow it (D <= 64), so one wave's row loads overlap the other's
// matrix steps.
__host__ __device__ constexpr int gather_waves_per_simd(int DP) { return DP <= 64 ? 2 : 1; }

template <int DP>
__global__ __attribute__((amdgpu_flat_work_group_size(64 * kGatherWaves, 64 * kGatherWaves),
                          amdgpu_waves_per_eu(gather_waves_per_simd(DP), gather_waves_per_simd(DP))))
void diag_accum_gather(const float* __restrict__ X, int64_t ldx, int64_t N, int D,
                       const bf16x8* __restrict__ mu3, const double* __restrict__ kc_x6lin, int KB, int KP,
                       const double* __restrict__ rowstat, const uint2* __restrict__ need, int nslab,
                       int64_t rows_per_slab, float* __restrict__ part_mu, float* __restrict__ part_sq,
                       float* __restrict__ part_nk, int dense, ProbeSel sel) {
  constexpr int NQ = DP / 8;      // chunks of 8 dimensions (16 features)
  constexpr int NQH = NQ / 2;
  constexpr int NJ = DP / 32;
  constexpr int RS = gather_rs(DP);
  constexpr int BLK = NQ * 4 * 64;
  static_assert(NQ % 2 == 0, "two halves of chunks");
  // The stored branch's diag_accum_ljt takes the call when the probe selects it.
  if (probe_selects(sel)) return;

  extern __shared__ __align__(16) unsigned char lds_raw[];
  unsigned char* lp = lds_raw;
  bf16x8* mu_l = reinterpret_cast<bf16x8*>(lp);  lp += (size_t)BLK * sizeof(bf16x8);
  float* xt_all = reinterpret_cast<float*>(lp);  lp += (size_t)kGatherWaves * 32 * RS * 4;
  double* rs_all = reinterpret_cast<double*>(lp); lp += (size_t)kGatherWaves * 32 * sizeof(double);
  int* q_all = reinterpret_cast<int*>(lp);

  const int tid = threadIdx.x, lane = tid & 63;
  const int wave = __builtin_amdgcn_readfirstlane(tid >> 6);
  const int c = lane & 31, g = lane >> 5;
  int sg, kb;
  if (!gather_item(blockIdx.x, gather_groups(nslab), KB, sg, kb)) return;   // uniform over the workgroup
  for (int idx = tid; idx < BLK; idx += 64 * kGatherWaves) mu_l[idx] = mu3[(int64_t)kb * BLK + idx];
  __syncthreads();
  const int slab = sg * kGatherWaves + wave;
  if (slab >= nslab) return;   // no barrier follows

  float* xt = xt_all + wave * 32 * RS;
  double* rs_l = rs_all + wave * 32;
  int* q_l = q_all + wave * 64;
  const double Cc = kc_x6lin[(int64_t)kb * 32 + c];

  const int64_t r_begin = (int64_t)slab * rows_per_slab;
  int64_t r_end = r_begin + rows_per_slab;
  if (r_end > N) r_end = N;
  const int64_t t_begin = r_begin / 32, t_end = cdiv(r_end, 32);

  auto words = [&](int64_t tb) -> unsigned {
    const int64_t t = tb + lane;
    if (t >= t_end) return 0u;
    const uint2 w = need[t * KB + kb];
    return w.x | w.y;
  };
  int64_t tb = t_begin;
  unsigned mword = words(tb), mnext = words(tb + 64);
  int jn = 0;
  int qh = 0, qt = 0;
  auto take = [&](int& e) -> int {
    queue_fill<(DP > 32)>(words, tb, t_begin, t_end, mword, mnext, jn, qt, qh, lane, c, g, q_l);
    const int cnt = qt - qh < 32 ? qt - qh : 32;
    asm volatile("s_waitcnt lgkmcnt(0)" ::: "memory");
    e = c < cnt ? q_l[(qh + c) & 63] : -1;
    qh += cnt;
    return cnt;
  };

  // The tile in flight: lane (c, g) holds row c's dimensions 8q + 4g .. +3.  The rows
  // come through resources over the slab (a lane without a row reads zeros and makes
  // no access, so the loads issue back to back): X so while D fills whole chunks and
  // the slab spans under 2 GiB (uniform), else load_row4.
  f32x4 raw[NQ];
  double rst;
  const int64_t slab_bytes = (r_end - r_begin) * ldx * (int64_t)sizeof(float);
  const bool xbuf = D == DP && slab_bytes <= ((int64_t)1 << 31) - 256;
  const buf_rsrc xres = make_rsrc(X + r_begin * ldx, xbuf ? (uint32_t)slab_bytes : 0u);
  const buf_rsrc rres = make_rsrc(rowstat + r_begin, (uint32_t)((r_end - r_begin) * sizeof(double)));
  auto issue = [&](int e) {
    const bool ok = e >= 0;
    if (xbuf) {
      const int off = buf_off(ok ? (int)((int64_t)e * ldx * (int64_t)sizeof(float)) + 16 * g : kBufOob);
#pragma unroll
      for (int q = 0; q < NQ; ++q)
        raw[q] = __builtin_bit_cast(f32x4, __builtin_amdgcn_raw_buffer_load_b128(xres, off, 32 * q, 0));
    } else {
      const int64_t row = r_begin + (ok ? e : 0);
#pragma unroll
      for (int q = 0; q < NQ; ++q) raw[q] = load_row4(X, ldx, row, 8 * q + 4 * g, D, ok);
    }
    const double z = buf_load_f64(rres, buf_off(ok ? e * (int)sizeof(double) : kBufOob));
    rst = ok ? z : INFINITY;
  };

  f32x16 accx[NJ], accq[NJ];
#pragma unroll
  for (int j = 0; j < NJ; ++j) {
    accx[j] = zero16();
    accq[j] = zero16();
  }
  float nk = 0.0f;
  const bf16x8 ones = x6c_ones(lane);

  int e;
  int cnt = take(e);
  if (cnt > 0) issue(e);
  while (cnt > 0) {
    asm volatile("s_waitcnt lgkmcnt(0)" ::: "memory");   // the previous tile's LDS reads are done
#pragma unroll
    for (int q = 0; q < NQ; ++q) *reinterpret_cast<f32x4*>(xt + c * RS + 8 * q + 4 * g) = raw[q];
    if (g == 0) rs_l[c] = rst;
    int en;
    const int cnt_next = take(en);
    if (cnt_next > 0) issue(en);
    asm volatile("s_waitcnt lgkmcnt(0)" ::: "memory");

    // [x^2, x] of chunk q, split three ways (pass 1's B operand, here the A operand).
    auto loadX = [&](int q, bf16x8 (&xa)[3]) {
      const f32x4 x = *reinterpret_cast<const f32x4*>(xt + c * RS + 8 * q + 4 * g);
      split3_bf16(x * x, x, xa);
    };
    const f32x16 s0 = x6c_tile_rows_fn<NQH, 2>(loadX, ones, [&](int q, int t) { return mu_l[(q * 4 + t) * 64 + lane]; });
    const f32x16 s1 = x6c_tile_rows_fn<NQH, 2>([&](int q, bf16x8 (&xa)[3]) { loadX(NQH + q, xa); }, ones,
                                               [&](int q, int t) { return mu_l[((NQH + q) * 4 + t) * 64 + lane]; });
    float r[16];
#pragma unroll
    for (int i = 0; i < 16; ++i) {
      const double ll = Cc + (double)(s0[i] + s1[i]);
      const float rv = fast_exp2((float)(ll - rs_l[acc_row(i, g)]));
      r[i] = rv;
      nk += rv;
    }
    // r = r1 + r2 + r3 (exact), as A operands of the two 16-row steps.
    bf16x8 a1[2], a2[2], a3[2];
    {
      float d1[16], d2[16];
#pragma unroll
      for (int i = 0; i < 16; ++i) {
        d1[i] = r[i] - (float)(__bf16)r[i];
        d2[i] = d1[i] - (float)(__bf16)d1[i];
      }
      acc_to_row_operands(r, a1);
      acc_to_row_operands(d1, a2);
      acc_to_row_operands(d2, a3);
    }
#pragma unroll
    for (int p = 0; p < 2; ++p) {
      bool any = false;
#pragma unroll
      for (int i = 8 * p; i < 8 * p + 8; ++i) any = any || r[i] != 0.0f;
      if (!dense && __builtin_amdgcn_ballot_w64(any) == 0) continue;
      // B operands: rows 16p + 8g + e of column 32j + c, and their squares.
      const float* xb = xt + (16 * p + 8 * g) * RS + c;
#pragma unroll
      for (int j = 0; j < NJ; ++j) {
        float v[8];
#pragma unroll
        for (int e = 0; e < 8; ++e) v[e] = xb[e * RS + 32 * j];
        bf16x8 bx[3], bq[3];
        split3_bf16(f32x4{v[0], v[1], v[2], v[3]}, f32x4{v[4], v[5], v[6], v[7]}, bx);
        split3_bf16(f32x4{v[0] * v[0], v[1] * v[1], v[2] * v[2], v[3] * v[3]},
                    f32x4{v[4] * v[4], v[5] * v[5], v[6] * v[6], v[7] * v[7]}, bq);
        accx[j] = mfma_bf16(a3[p], bx[0], accx[j]);
        accx[j] = mfma_bf16(a2[p], bx[1], accx[j]);
        accx[j] = mfma_bf16(a1[p], bx[2], accx[j]);
        accx[j] = mfma_bf16(a2[p], bx[0], accx[j]);
        accx[j] = mfma_bf16(a1[p], bx[1], accx[j]);
        accx[j] = mfma_bf16(a1[p], bx[0], accx[j]);
        accq[j] = mfma_bf16(a3[p], bq[0], accq[j]);
        accq[j] = mfma_bf16(a2[p], bq[1], accq[j]);
        accq[j] = mfma_bf16(a1[p], bq[2], accq[j]);
        accq[j] = mfma_bf16(a2[p], bq[0], accq[j]);
        accq[j] = mfma_bf16(a1[p], bq[1], accq[j]);
        accq[j] = mfma_bf16(a1[p], bq[0], accq[j]);
      }
    }
    cnt = cnt_next;
  }

  nk += __shfl_xor(nk, 32);
  const int64_t kbase = (int64_t)slab * KP + (int64_t)kb * 32;
#pragma unroll
  for (int j = 0; j < NJ; ++j) {
#pragma unroll
    for (int i = 0; i < 16; ++i) {
      part_mu[(kbase + acc_row(i, g)) * DP + 32 * j + c] = accx[j][i];
      part_sq[(kbase + acc_row(i, g)) * DP + 32 * j + c] = accq[j][i];
    }
  }
  if (g == 0) part_nk[kbase + c] = nk;
}

// ---------------------------------------------------------------------------
// Pass 2 of the stored branch (FGMM_FLAG_STORE_LOGJOINT_AUTO, D <= 96): pass 1 left
// per 32-row tile every block's log-joint tile, the rows' features [x^2 | x] in three
// bf16 parts and logZ2 as (hi, lo) float pairs.  Per 16-row step, r is split in three
// bf16 parts as well and r^T [x^2 | x] is accumulated from the six products of
// significance at least 2^-16, smallest first (r3 f1, r2 f2, r1 f3, r2 f1, r1 f2,
// r1 f1), as the gathering pass does: the sig identity in diag_reduce needs an fp32
// step's accuracy of these moments.
//
// Grid over (row slab x group of 8 component blocks); wave w owns block 8 cg + w and
// its partial of the slab; the workgroups of a slab run on one XCD, so the feature
// parts come from HBM once.  Stages of one tile each (its feature parts, the 8
// blocks' log-joint tiles, the logZ2 pairs), all filled by buffer-to-LDS loads,
// three where they fit in LDS (D <= 32) and two above: at step t the workgroup
// issues tile t + NS - 1's loads, computes tile t and waits for tile t + 1's.  Every
// wave issues the same number of loads per tile (loads that only keep the count go
// out of range into a pad line), so that wait is a fixed count.  A wave skips a
// tile whose need words are both zero; otherwise it exponentiates the whole tile
// with no per-row select: a row whose need bits are clear has l < logZ2 - kLjNeedGap
// in every component of the block (pass 1's bounds are rounded up), so 2^(l - logZ2)
// is exactly 0 in fp32, and a row past N has the pair (+inf, 0).  `sel` is the
// probe's selector: the kernel returns unless it selects the stored branch.
// ---------------------------------------------------------------------------
constexpr int kLjdWaves = 8;

template <int DP>
struct LjdShape {
  static constexpr int RS = ljd_rs(DP);
  static constexpr int XB = (int)ljd_xsplit_bytes(DP);      // a tile's feature parts
  static constexpr int XP = XB / 16;                         // their 16-byte pieces
  static constexpr int XQ = (XP + 64 * kLjdWaves - 1) / (64 * kLjdWaves);
  static constexpr int LJB = kLjdWaves * kLjTile * 4;        // the 8 blocks' log-joint tiles
  static constexpr int OFF_X = LJB, OFF_Z = LJB + XB;
  static constexpr int STAGE = LJB + XB + 32 * 8;
  static constexpr int NS = (size_t)3 * STAGE + 1024 <= kMaxLds ? 3 : 2;
  static constexpr int OFF_PAD = NS * STAGE;
  static constexpr size_t lds = (size_t)OFF_PAD + 1024;
  // Loads of every wave per tile: XQ of feature parts, 4 of its log-joint tile, 1 of
  // logZ2 pairs (wave 0's; an out-of-range one elsewhere).
  static constexpr int NLOADS = XQ + 4 + 1;
};
__host__ inline int64_t ljd_grid(int nslab, int ncg) { return (int64_t)8 * cdiv(nslab, 8) * ncg; }

template <int DP>
__global__ __attribute__((amdgpu_flat_work_group_size(64 * kLjdWaves, 64 * kLjdWaves), amdgpu_waves_per_eu(2, 2)))
void diag_accum_ljt(const float* __restrict__ lj, const __bf16* __restrict__ xsplit, const float2* __restrict__ zpair,
                    int64_t N, const uint2* __restrict__ need, ProbeSel sel, int KB, int KP, int nslab,
                    int64_t rows_per_slab, int ncg, float* __restrict__ part_mu, float* __restrict__ part_sq,
                    float* __restrict__ part_nk) {
  using SH = LjdShape<DP>;
  static_assert(SH::XP % 64 == 0, "whole waves of feature pieces");
  static_assert(SH::lds <= kMaxLds, "stages exceed LDS");
  constexpr int NJ = 2 * DP / 32;   // 32-feature column tiles
  constexpr int RS = SH::RS;
  constexpr int NS = SH::NS;
  constexpr int NL = SH::NLOADS;
  if (!probe_selects(sel)) return;

  extern __shared__ __align__(16) unsigned char lds_raw[];
  const int tid = threadIdx.x, lane = tid & 63;
  const int wave = __builtin_amdgcn_readfirstlane(tid >> 6);
  const int c = lane & 31, g = lane >> 5;
  // Workgroup -> (slab, component group): the ncg groups of slab s run on XCD s % 8.
  const int xcd = blockIdx.x & 7, item = blockIdx.x >> 3;
  const int slab = (item / ncg) * 8 + xcd, cg = item % ncg;
  if (slab >= nslab) return;   // uniform over the workgroup
  const int kb = cg * kLjdWaves + wave;
  const bool active = kb < KB;

  const int64_t r_begin = (int64_t)slab * rows_per_slab;
  int64_t r_end = r_begin + rows_per_slab;
  if (r_end > N) r_end = N;
  const int ntiles = r_end > r_begin ? (int)cdiv(r_end - r_begin, 32) : 0;
  const int64_t tile0 = r_begin >> 5;   // rows_per_slab is a multiple of 32

  f32x16 acc[NJ];
#pragma unroll
  for (int j = 0; j < NJ; ++j) acc[j] = zero16();
  float nk = 0.0f;

  // The wave's need words of tile t (0 past the slab or the blocks), ORed.
  auto mword = [&](int t) -> unsigned {
    const bool ok = active && t < ntiles;
    const uint2 v = need[ok ? (tile0 + t) * KB + kb : 0];
    return ok ? (v.x | v.y) : 0u;
  };
  unsigned char* const pad = lds_raw + SH::OFF_PAD;
  auto issue = [&](int t, auto stage_tag, unsigned m) __attribute__((always_inline)) {
    constexpr int S = decltype(stage_tag)::value;
    unsigned char* st = lds_raw + (size_t)S * SH::STAGE;
    const bool in = t < ntiles;
    const int64_t tg = tile0 + t;
    const DmaSrc xsrc = dma_src(in ? reinterpret_cast<const unsigned char*>(xsplit) + tg * SH::XB
                                   : reinterpret_cast<const unsigned char*>(xsplit),
                                in ? (uint32_t)SH::XB : 0u);
#pragma unroll
    for (int q = 0; q < SH::XQ; ++q) {
      if (q * 64 * kLjdWaves + wave * 64 < SH::XP)
        lds_dma16(xsrc, st + SH::OFF_X + (q * 64 * kLjdWaves + wave * 64) * 16,
                  (q * 64 * kLjdWaves + tid) * 16, 0);
      else
        lds_dma16(xsrc, pad, kBufOob, 0);
    }
    const DmaSrc lsrc = dma_src(m ? lj + (tg * KB + kb) * kLjTile : lj, m ? (uint32_t)(kLjTile * 4) : 0u);
#pragma unroll
    for (int q = 0; q < 4; ++q) lds_dma16(lsrc, st + wave * kLjTile * 4 + q * 1024, (q * 64 + lane) * 16, 0);
    if (wave == 0) {
      const DmaSrc zsrc = dma_src(zpair + tg * 32 * (in ? 1 : 0), in ? (uint32_t)(32 * sizeof(float2)) : 0u);
      if (lane < 16) lds_dma16(zsrc, st + SH::OFF_Z, lane * 16, 0);
    } else {
      lds_dma16(lsrc, pad, kBufOob, 0);
    }
  };
  // Tile t in stage S: per 16-row half p, r in three parts (registers 8p .. 8p + 7 of
  // the accumulator layout: lane = component, rows acc_row), then the six products
  // for each column tile.
  auto compute = [&](auto stage_tag) __attribute__((always_inline)) {
    constexpr int S = decltype(stage_tag)::value;
    int sb = S * SH::STAGE;
    asm volatile("" : "+s"(sb));
    int lofs = sb + wave * kLjTile * 4 + 4 * c + 4 * 32 * 4 * g;
    int zofs = sb + SH::OFF_Z + 4 * 8 * g;
    asm volatile("" : "+v"(lofs), "+v"(zofs));
    const float* lt = reinterpret_cast<const float*>(lds_raw + lofs);
    const f32x4* zt = reinterpret_cast<const f32x4*>(lds_raw + zofs);
    const __bf16* xt = reinterpret_cast<const __bf16*>(lds_raw + sb + SH::OFF_X);
#pragma unroll
    for (int p = 0; p < 2; ++p) {
      float r[8];
#pragma unroll
      for (int jj = 0; jj < 2; ++jj) {
        const int j = 2 * p + jj;   // registers 4j .. 4j + 3: rows 8j + 4g .. + 3
        const f32x4 z01 = zt[4 * j], z23 = zt[4 * j + 1];
        const float zh[4] = {z01[0], z01[2], z23[0], z23[2]}, zl[4] = {z01[1], z01[3], z23[1], z23[3]};
#pragma unroll
        for (int e = 0; e < 4; ++e) {
          const float rv = fast_exp2((lt[(8 * j + e) * 32] - zh[e]) - zl[e]);
          r[4 * jj + e] = rv;
          nk += rv;
        }
      }
      bf16x8 a1, a2, a3;
      acc_to_row_operands_split3(r, a1, a2, a3);
#pragma unroll
      for (int j = 0; j < NJ; ++j) {
        const bf16x8 f1 = lds_rows_operand(xt, RS, 16 * p, 32 * j, lane);
        const bf16x8 f2 = lds_rows_operand(xt + 32 * RS, RS, 16 * p, 32 * j, lane);
        const bf16x8 f3 = lds_rows_operand(xt + 64 * RS, RS, 16 * p, 32 * j, lane);
        acc[j] = mfma_bf16(a3, f1, acc[j]);
        acc[j] = mfma_bf16(a2, f2, acc[j]);
        acc[j] = mfma_bf16(a1, f3, acc[j]);
        acc[j] = mfma_bf16(a2, f1, acc[j]);
        acc[j] = mfma_bf16(a1, f2, acc[j]);
        acc[j] = mfma_bf16(a1, f1, acc[j]);
      }
    }
  };

  unsigned mk[NS];
  unsigned mnext = 0u;
  // Step t, stage S = t mod NS: issue tile t + NS - 1 (its stage was freed by the last
  // barrier), compute tile t, wait for tile t + 1's stage (the loads issued after it
  // are those of tiles t + 2 ..), barrier.
  auto step = [&](int t, auto stage_tag) __attribute__((always_inline)) {
    constexpr int S = decltype(stage_tag)::value;
    constexpr int SI = (S + NS - 1) % NS;
    mk[SI] = mnext;
    issue(t + NS - 1, std::integral_constant<int, SI>{}, mnext);
    mnext = mword(t + NS);
    if (mk[S] != 0u) compute(stage_tag);
    vm_wait<(NS - 2) * NL>();
    __syncthreads();
  };
  if (ntiles > 0) {
#pragma unroll
    for (int u = 0; u < NS - 1; ++u) mk[u] = mword(u);
    issue(0, std::integral_constant<int, 0>{}, mk[0]);
    if constexpr (NS == 3) issue(1, std::integral_constant<int, 1>{}, mk[1]);
    mnext = mword(NS - 1);
    vm_wait<(NS - 2) * NL>();   // tile 0's stage
    __syncthreads();
  }
  using S0 = std::integral_constant<int, 0>;
  using S1 = std::integral_constant<int, 1>;
  using S2 = std::integral_constant<int, 2 % NS>;
  for (int t = 0; t < ntiles; t += NS) {
    step(t, S0{});
    if (t + 1 >= ntiles) break;
    step(t + 1, S1{});
    if constexpr (NS == 3) {
      if (t + 2 >= ntiles) break;
      step(t + 2, S2{});
    }
  }
  vm_wait<0>();   // no buffer-to-LDS load outlives the workgroup

  if (active) {
    nk += __shfl_xor(nk, 32);
    const int64_t kbase = (int64_t)slab * KP + (int64_t)kb * 32;
    // Column f of the feature parts is x^2 (f % 8 < 4) or x of dimension
    // 8 (f / 16) + 4 ((f / 8) % 2) + f % 4.
#pragma unroll
    for (int j = 0; j < NJ; ++j) {
      const int f = 32 * j + c;
      const int dim = 8 * (f >> 4) + 4 * ((f >> 3) & 1) + (f & 3);
      float* dst = ((f & 7) < 4 ? part_sq : part_mu) + dim;
#pragma unroll
      for (int i = 0; i < 16; ++i) dst[(kbase + acc_row(i, g)) * DP] = acc[j][i];
    }
    if (g == 0) part_nk[kbase + c] = nk;
  }
}

// ---------------------------------------------------------------------------
// Pass 2 of the default plan above D = 128: the isotropic iso_accum_drange's
// structure over the diagonal features.  One workgroup of four waves per (row slab,
// component block, range of up to kDrange dimensions); the waves queue the same
// needed rows (either half's word); per 32 queued rows wave w forms chain w of S
// over the chunks q = w, w + 4, ... of all of D (x6c_tile_rows' products and order
// on [x^2, x]) and stores the fp32 rows of its chunks in the range to the LDS tile;
// the chains meet in LDS and every wave adds them as pass 1 does, so the log-joint
// C'_k + S equals pass 1's bit for bit; r = 2^(ll2 - logZ2), and each wave
// accumulates r^T X and r^T X^2 for a quarter of the range's 32-column tiles as six
// split-bf16 products per 16 rows (the sig identity in diag_reduce cancels, so these
// moments keep an fp32 step's accuracy).  Wave 0 of the first range also sums Nk.
// ---------------------------------------------------------------------------
__global__ __attribute__((amdgpu_flat_work_group_size(64 * kCtWaves, 64 * kCtWaves), amdgpu_waves_per_eu(1, 1)))
void diag_accum_drange(const float* __restrict__ X, int64_t ldx, int64_t N, int D, int NQ, int DP,
                       const bf16x8* __restrict__ mu3, const double* __restrict__ kc_x6lin, int KB, int KP,
                       const double* __restrict__ rowstat, const uint2* __restrict__ need, int nslab,
                       int64_t rows_per_slab, int ndr, float* __restrict__ part_mu, float* __restrict__ part_sq,
                       float* __restrict__ part_nk, int dense) {
  // Workgroup -> (block, slab, range), blocks contiguous per XCD.
  const int64_t total = (int64_t)KB * nslab * ndr;
  const int64_t per = cdiv(total, 8);
  const int64_t item = (int64_t)(blockIdx.x & 7) * per + (blockIdx.x >> 3);
  if (item >= total) return;   // uniform over the workgroup
  const int dr = (int)(item % ndr);
  const int slab = (int)((item / ndr) % nslab);
  const int kb = (int)(item / ((int64_t)ndr * nslab));

  const int RS = drange_rs(DP < kDrange ? DP : kDrange);
  extern __shared__ __align__(16) unsigned char lds_raw[];
  unsigned char* lp = lds_raw;
  float* xt = reinterpret_cast<float*>(lp);       lp += (size_t)32 * RS * sizeof(float);   // [row][RS]
  float* ex = reinterpret_cast<float*>(lp);       lp += (size_t)kCtWaves * 16 * 64 * sizeof(float);
  double* rs_l = reinterpret_cast<double*>(lp);   lp += (size_t)32 * sizeof(double);
  int* q_all = reinterpret_cast<int*>(lp);

  const int tid = threadIdx.x, lane = tid & 63;
  const int wave = __builtin_amdgcn_readfirstlane(tid >> 6);
  const int c = lane & 31, g = lane >> 5;
  int* q_l = q_all + wave * 64;

  const int d0 = dr * kDrange;
  const int DR = DP - d0 < kDrange ? DP - d0 : kDrange;   // a multiple of 64
  const int q_lo = d0 / 8, q_hi = (d0 + DR) / 8;           // chunks of the range
  const int njr = DR / 32;
  const int tj = (njr + kCtWaves - 1) / kCtWaves;
  const int j0 = wave * tj;
  const int nj = njr - j0 < tj ? (njr - j0 > 0 ? njr - j0 : 0) : tj;   // this wave's column tiles
  const int nqw = NQ / kCtWaves;                                       // chunks per wave

  const double Cc = kc_x6lin[(int64_t)kb * 32 + c];

  const int64_t r_begin = (int64_t)slab * rows_per_slab;
  int64_t r_end = r_begin + rows_per_slab;
  if (r_end > N) r_end = N;
  const int64_t t_begin = r_begin / 32, t_end = cdiv(r_end, 32);

  auto words = [&](int64_t tb) -> unsigned {
    const int64_t t = tb + lane;
    if (t >= t_end) return 0u;
    const uint2 w = need[t * KB + kb];
    return w.x | w.y;
  };
  int64_t tb = t_begin;
  unsigned mword = words(tb), mnext = words(tb + 64);
  int jn = 0;
  int qh = 0, qt = 0;
  auto take = [&](int& e) -> int {
    queue_fill<true>(words, tb, t_begin, t_end, mword, mnext, jn, qt, qh, lane, c, g, q_l);
    const int cnt = qt - qh < 32 ? qt - qh : 32;
    asm volatile("s_waitcnt lgkmcnt(0)" ::: "memory");
    e = c < cnt ? q_l[(qh + c) & 63] : -1;
    qh += cnt;
    return cnt;
  };

  // Chunk i of this wave (chunk q = wave + 4 i): the rows' dimensions 8q + 4g .. + 3
  // and mu's four operands of the chunk.
  const buf_rsrc mrs = make_rsrc(mu3 + (int64_t)kb * NQ * 4 * 64, (uint32_t)((int64_t)NQ * 4 * 64 * sizeof(bf16x8)));
  auto issue = [&](int i, int e, f32x4& x, bf16x8 (&m)[4]) __attribute__((always_inline)) {
    const int q = wave + kCtWaves * i;
    const bool ok = e >= 0;
    x = load_row4(X, ldx, r_begin + (ok ? e : 0), 8 * q + 4 * g, D, ok);
#pragma unroll
    for (int t = 0; t < 4; ++t)
      m[t] = __builtin_bit_cast(bf16x8, __builtin_amdgcn_raw_buffer_load_b128(
                                            mrs, lane * (int)sizeof(bf16x8), (q * 4 + t) * 64 * (int)sizeof(bf16x8), 0));
  };
  f32x4 xr[2];
  bf16x8 mr[2][4];
  double rst = INFINITY;
  auto start = [&](int e) __attribute__((always_inline)) {
    issue(0, e, xr[0], mr[0]);
    if (nqw > 1) issue(1, e, xr[1], mr[1]);
    if (wave == 0) {
      const double z = rowstat[r_begin + (e >= 0 ? e : 0)];   // a row of the slab: no branch
      rst = e >= 0 ? z : INFINITY;
    }
  };

  f32x16 accx[kDrTiles], accq[kDrTiles];
#pragma unroll
  for (int j = 0; j < kDrTiles; ++j) {
    accx[j] = zero16();
    accq[j] = zero16();
  }
  float nk = 0.0f;
  const bf16x8 ones = x6c_ones(lane);

  int e;
  int cnt = take(e);
  if (cnt > 0) start(e);
  while (cnt > 0) {
    f32x16 cs = zero16();
    auto chunk = [&](int i, const f32x4& x, const bf16x8 (&m)[4]) __attribute__((always_inline)) {
      const int q = wave + kCtWaves * i;
      if (q >= q_lo && q < q_hi) *reinterpret_cast<f32x4*>(xt + c * RS + 8 * (q - q_lo) + 4 * g) = x;
      bf16x8 xa[3];
      split3_bf16(x * x, x, xa);
#pragma unroll
      for (int step = 0; step < 7; ++step) {
        const bf16x8 B = step == 0 ? m[1] : step == 1 ? m[2] : step <= 3 ? m[0] : step == 4 ? m[1]
                       : step == 5 ? m[3] : m[0];
        const bf16x8 A = step == 0 ? xa[1] : step == 1 ? xa[0] : step == 2 ? xa[2] : step == 3 ? xa[1]
                       : step == 4 ? xa[0] : step == 5 ? ones : xa[0];
        cs = mfma_bf16(A, B, cs);
      }
    };
    for (int i = 0; i < nqw; i += 2) {
      chunk(i, xr[0], mr[0]);
      if (i + 2 < nqw) issue(i + 2, e, xr[0], mr[0]);
      if (i + 1 < nqw) {
        chunk(i + 1, xr[1], mr[1]);
        if (i + 3 < nqw) issue(i + 3, e, xr[1], mr[1]);
      }
    }
    float* exw = ex + wave * 16 * 64 + lane;
#pragma unroll
    for (int i = 0; i < 16; ++i) exw[i * 64] = cs[i];
    if (wave == 0 && g == 0) rs_l[c] = rst;
    int en;
    const int cnt_next = take(en);
    if (cnt_next > 0) start(en);
    lds_barrier();

    float r[16];
#pragma unroll
    for (int i = 0; i < 16; ++i) {
      const float S = ((ex[i * 64 + lane] + ex[(16 + i) * 64 + lane]) + ex[(32 + i) * 64 + lane]) +
                      ex[(48 + i) * 64 + lane];
      const double ll = Cc + (double)S;
      const float rv = fast_exp2((float)(ll - rs_l[acc_row(i, g)]));
      r[i] = rv;
      nk += rv;
    }
    // r^T [X | X^2] as diag_accum_gather forms it: six split-bf16 products per 16 rows.
    bf16x8 a1[2], a2[2], a3[2];
    {
      float d1[16], d2[16];
#pragma unroll
      for (int i = 0; i < 16; ++i) {
        d1[i] = r[i] - (float)(__bf16)r[i];
        d2[i] = d1[i] - (float)(__bf16)d1[i];
      }
      acc_to_row_operands(r, a1);
      acc_to_row_operands(d1, a2);
      acc_to_row_operands(d2, a3);
    }
#pragma unroll
    for (int p = 0; p < 2; ++p) {
      bool any = false;
#pragma unroll
      for (int i = 8 * p; i < 8 * p + 8; ++i) any = any || r[i] != 0.0f;
      if (!dense && __builtin_amdgcn_ballot_w64(any) == 0) continue;
      const float* xb = xt + (16 * p + 8 * g) * RS + c;
#pragma unroll
      for (int jj = 0; jj < kDrTiles; ++jj) {
        if (jj < nj) {
          float v[8];
#pragma unroll
          for (int e = 0; e < 8; ++e) v[e] = xb[e * RS + 32 * (j0 + jj)];
          bf16x8 bx[3], bq[3];
          split3_bf16(f32x4{v[0], v[1], v[2], v[3]}, f32x4{v[4], v[5], v[6], v[7]}, bx);
          split3_bf16(f32x4{v[0] * v[0], v[1] * v[1], v[2] * v[2], v[3] * v[3]},
                      f32x4{v[4] * v[4], v[5] * v[5], v[6] * v[6], v[7] * v[7]}, bq);
          accx[jj] = mfma_bf16(a3[p], bx[0], accx[jj]);
          accx[jj] = mfma_bf16(a2[p], bx[1], accx[jj]);
          accx[jj] = mfma_bf16(a1[p], bx[2], accx[jj]);
          accx[jj] = mfma_bf16(a2[p], bx[0], accx[jj]);
          accx[jj] = mfma_bf16(a1[p], bx[1], accx[jj]);
          accx[jj] = mfma_bf16(a1[p], bx[0], accx[jj]);
          accq[jj] = mfma_bf16(a3[p], bq[0], accq[jj]);
          accq[jj] = mfma_bf16(a2[p], bq[1], accq[jj]);
          accq[jj] = mfma_bf16(a1[p], bq[2], accq[jj]);
          accq[jj] = mfma_bf16(a2[p], bq[0], accq[jj]);
          accq[jj] = mfma_bf16(a1[p], bq[1], accq[jj]);
          accq[jj] = mfma_bf16(a1[p], bq[0], accq[jj]);
        }
      }
    }
    lds_barrier();   // the tile and the chains are free for the next rows
    e = en;
    cnt = cnt_next;
  }

  const int64_t kbase = (int64_t)slab * KP + (int64_t)kb * 32;
#pragma unroll
  for (int jj = 0; jj < kDrTiles; ++jj) {
    if (jj < nj) {
#pragma unroll
      for (int i = 0; i < 16; ++i) {
        const int64_t o = (kbase + acc_row(i, g)) * DP + d0 + 32 * (j0 + jj) + c;
        part_mu[o] = accx[jj][i];
        part_sq[o] = accq[jj][i];
      }
    }
  }
  if (dr == 0 && wave == 0) {
    nk += __shfl_xor(nk, 32);
    if (g == 0) part_nk[kbase + c] = nk;
  }
}

// Finish: one thread per (k, d); fixed-order fp64 sums over partials, then the
// sig identity in fp64.  Thread d == 0 also writes Nk.
template <bool WIDE>
__global__ __launch_bounds__(256) void diag_reduce(const float* __restrict__ part_mu,
                                                   const float* __restrict__ part_sq,
                                                   const float* __restrict__ part_nk, int npart, int KP,
                                                   int DP, int64_t K, int D, const float* __restrict__ mu,
                                                   int64_t ldmu, float* __restrict__ Nk,
                                                   float* __restrict__ mu_acc, float* __restrict__ sig_acc,
                                                   int accumulate) {
  // WIDE: one wave per (k, d) with the partials spread over its lanes (many partials).
  const int64_t idx = WIDE ? (int64_t)blockIdx.x * 4 + (threadIdx.x >> 6)
                           : (int64_t)blockIdx.x * blockDim.x + threadIdx.x;
  const int lane = threadIdx.x & 63;
  if (idx >= K * D) return;
  const int64_t k = idx / D;
  const int d = (int)(idx % D);
  auto sum = [&](const float* p, int64_t stride) {
    return WIDE ? wave_strided_sum(p, npart, stride, lane) : strided_sum(p, npart, stride);
  };
  const double sm = sum(part_mu + k * DP + d, (int64_t)KP * DP);
  const double sq = sum(part_sq + k * DP + d, (int64_t)KP * DP);
  const double nk = sum(part_nk + k, KP);
  if (WIDE && lane != 0) return;
  const double m = (double)mu[k * ldmu + d];
  const double sg = sq - 2.0 * m * sm + m * m * nk;
  float* om = mu_acc + k * D + d;
  float* os = sig_acc + k * D + d;
  *om = accumulate ? (float)((double)*om + sm) : (float)sm;
  *os = accumulate ? (float)((double)*os + sg) : (float)sg;
  if (d == 0) Nk[k] = accumulate ? (float)((double)Nk[k] + nk) : (float)nk;
}

// Atomic finish (FGMM_FLAG_ATOMIC_REDUCE): partial blockIdx.y of every (k, d) is added
// into the zeroed (or accumulated) outputs; the sig identity is formed per partial in
// fp64 and added in fp32.
__global__ __launch_bounds__(256) void diag_reduce_atomic(const float* __restrict__ part_mu,
                                                          const float* __restrict__ part_sq,
                                                          const float* __restrict__ part_nk, int KP, int DP,
                                                          int64_t K, int D, const float* __restrict__ mu,
                                                          int64_t ldmu, float* __restrict__ Nk,
                                                          float* __restrict__ mu_acc, float* __restrict__ sig_acc) {
  const int64_t idx = (int64_t)blockIdx.x * blockDim.x + threadIdx.x;
  if (idx >= K * D) return;
  const int64_t k = idx / D;
  const int d = (int)(idx % D);
  const int64_t pk = (int64_t)blockIdx.y * KP + k;
  const double sm = (double)part_mu[pk * DP + d];
  const double sq = (double)part_sq[pk * DP + d];
  const double nk = (double)part_nk[pk];
  const double m = (double)mu[k * ldmu + d];
  atomicAdd(mu_acc + k * D + d, (float)sm);
  atomicAdd(sig_acc + k * D + d, (float)(sq - 2.0 * m * sm + m * m * nk));
  if (d == 0) atomicAdd(Nk + k, (float)nk);
}

__global__ __launch_bounds__(256) void diag_fill(float* __restrict__ p, int64_t n, float v) {
  const int64_t i = (int64_t)blockIdx.x * blockDim.x + threadIdx.x;
  if (i < n) p[i] = v;
}

// Above D = 128: pass 1 is diag_lse_ctile for both plans; pass 2 of the default plan
// (any D) is diag_accum_drange, that of the stored plan (D <= 256) launch_passes'.
hipError_t launch_ctile(const DiagPlan& pl, const float* X, int64_t ldx, unsigned char* ws, float* logZ,
                        bool run1, bool run2, bool dense, hipStream_t stream) {
  const bf16x8* mu3 = reinterpret_cast<const bf16x8*>(ws + pl.off_mu3);
  double* rowstat = reinterpret_cast<double*>(ws + pl.off_rowstat);
  uint2* masks = reinterpret_cast<uint2*>(ws + pl.off_ljmask);
  const int NQ = pl.DP / 8;
  if (run1) {
    const bool exact = pl.rexact && !pl.lj;
    const int ctb = ctile_blocks(pl.DP);
    const size_t lds1 = lse_ctile_base(ctb) + (exact ? (size_t)kCtWaves * 2 * 32 * pl.KB * 2 : 0);
    auto kern = pl.lj ? (ctb == 2 ? &diag_lse_ctile<kLjmStore, 2> : &diag_lse_ctile<kLjmStore, 4>)
                      : (ctb == 2 ? &diag_lse_ctile<kLjmNeed, 2> : &diag_lse_ctile<kLjmNeed, 4>);
    hipError_t e = hipFuncSetAttribute(reinterpret_cast<const void*>(kern),
                                       hipFuncAttributeMaxDynamicSharedMemorySize, (int)lds1);
    if (e != hipSuccess) return e;
    hipLaunchKernelGGL(kern, dim3((unsigned)cdiv(pl.N, 32 * kCtWaves)), dim3(64 * kCtWaves), lds1, stream, X,
                       ldx, pl.N, (int)pl.D, NQ, mu3, reinterpret_cast<const double*>(ws + pl.off_kcx6), pl.KB,
                       logZ, rowstat, pl.lj ? reinterpret_cast<float*>(ws + pl.off_lj) : nullptr, masks,
                       dense ? 1 : 0, exact ? 1 : 0);
  }
  if (run2 && !pl.lj) {
    const size_t lds2 = accum_drange_lds_bytes(pl.DP < kDrange ? pl.DP : kDrange);
    hipError_t e = hipFuncSetAttribute(reinterpret_cast<const void*>(&diag_accum_drange),
                                       hipFuncAttributeMaxDynamicSharedMemorySize, (int)lds2);
    if (e != hipSuccess) return e;
    const int64_t items = (int64_t)pl.KB * pl.nslab * pl.ndr;
    hipLaunchKernelGGL(diag_accum_drange, dim3((unsigned)(8 * cdiv(items, 8))), dim3(64 * kCtWaves), lds2,
                       stream, X, ldx, pl.N, (int)pl.D, NQ, pl.DP, mu3,
                       reinterpret_cast<const double*>(ws + pl.off_kcx6lin), pl.KB, pl.KP, rowstat, masks,
                       pl.nslab, pl.rows_per_slab, pl.ndr, reinterpret_cast<float*>(ws + pl.off_part_mu),
                       reinterpret_cast<float*>(ws + pl.off_part_sq), reinterpret_cast<float*>(ws + pl.off_part_nk),
                       dense ? 1 : 0);
  }
  return hipGetLastError();
}

// Up to D = 128 both plans; above, the stored plan's pass 2 (pass 1 is launch_ctile's).
template <int DP>
hipError_t launch_passes(const DiagPlan& pl, const float* X, int64_t ldx, unsigned char* ws,
                         float* logZ, bool run1, bool run2, bool dense, hipStream_t stream) {
  double* rowstat = reinterpret_cast<double*>(ws + pl.off_rowstat);
  float* lj = pl.lj ? reinterpret_cast<float*>(ws + pl.off_lj) : nullptr;
  float* ljmax = pl.lj_sparse ? reinterpret_cast<float*>(ws + pl.off_ljmax) : nullptr;
  uint2* ljmask = pl.lj_sparse ? reinterpret_cast<uint2*>(ws + pl.off_ljmask) : nullptr;
  unsigned* ljcount = pl.lj_sparse ? reinterpret_cast<unsigned*>(ws + pl.off_ljcount) : nullptr;
  float* pmu = reinterpret_cast<float*>(ws + pl.off_part_mu);
  float* psq = reinterpret_cast<float*>(ws + pl.off_part_sq);
  float* pnk = reinterpret_cast<float*>(ws + pl.off_part_nk);
  // FGMM_FLAG_STORE_LOGJOINT_AUTO: the probe's counts, which pass 1 and both pass-2
  // kernels read to select the stored branch.
  unsigned* probe = pl.autolj ? reinterpret_cast<unsigned*>(ws + pl.off_probe) : nullptr;
  const ProbeSel psel = probe ? ProbeSel{probe, pl.nprobe, probe_min_pairs(pl.N, pl.nprobe, pl.KB)}
                              : ProbeSel{nullptr, 0, 0};
  if (run1) {
    const unsigned nblk1 = (unsigned)cdiv(pl.N, 32 * kWaves);
    if constexpr (diag_uses_x6(DP)) {
      if constexpr (ljd_applies(DP)) {
        if (pl.autolj)
          hipLaunchKernelGGL((diag_store_probe<DP>), dim3((unsigned)pl.nprobe), dim3(64 * kProbeWaves), 0, stream,
                             X, ldx, pl.N, (int)pl.D, reinterpret_cast<const bf16x8*>(ws + pl.off_mu3),
                             reinterpret_cast<const double*>(ws + pl.off_kcx6), pl.KB, pl.nprobe, probe);
      }
      const size_t lds1 = x6_lds_bytes<DP>() + (pl.rexact ? (size_t)kAccWaves * 32 * pl.KB * 2 : 0);
      uint2* masks = pl.need ? reinterpret_cast<uint2*>(ws + pl.off_ljmask) : ljmask;
      auto launch1 = [&](auto kern) -> hipError_t {
        if (lds1 > 65536) {
          hipError_t e = hipFuncSetAttribute(reinterpret_cast<const void*>(kern),
                                             hipFuncAttributeMaxDynamicSharedMemorySize, (int)lds1);
          if (e != hipSuccess) return e;
        }
        hipLaunchKernelGGL(kern, dim3(nblk1), dim3(kAccThreads), lds1, stream, X, ldx, pl.N, (int)pl.D,
                           reinterpret_cast<const bf16x8*>(ws + pl.off_mu3),
                           reinterpret_cast<const double*>(ws + pl.off_kcx6), pl.KB, logZ, rowstat, lj,
                           ljmax, reinterpret_cast<unsigned*>(masks), ljcount, dense ? 1 : 0, pl.rexact ? 1 : 0,
                           psel, pl.autolj ? reinterpret_cast<float*>(ws + pl.off_lj) : nullptr,
                           reinterpret_cast<__bf16*>(ws + pl.off_xsplit),
                           reinterpret_cast<float2*>(ws + pl.off_zpair));
        return hipSuccess;
      };
      hipError_t e1 = launch1(pl.lj ? &diag_lse_x6<DP, kLjmStore> : &diag_lse_x6<DP, kLjmNeed>);
      if (e1 != hipSuccess) return e1;
      if constexpr (ljd_applies(DP)) {
        if (pl.autolj) {
          e1 = launch1(&diag_lse_x6<DP, kLjmNeed, true>);
          if (e1 != hipSuccess) return e1;
        }
      }
    } else {
      return hipErrorInvalidValue;   // launch_ctile runs pass 1 above D = 128
    }
  }
  if (!run2) return hipGetLastError();
  const dim3 grid2((unsigned)(pl.nslab * pl.ncg));
  if constexpr (diag_uses_x6(DP)) {
    if (pl.need) {
      // With the stored branch both pass-2 kernels are launched over the same slabs and
      // partials; the probe's selector lets one of them run.
      if constexpr (ljd_applies(DP)) {
        if (pl.autolj) {
          using SH = LjdShape<DP>;
          hipError_t ej = hipFuncSetAttribute(reinterpret_cast<const void*>(&diag_accum_ljt<DP>),
                                              hipFuncAttributeMaxDynamicSharedMemorySize, (int)SH::lds);
          if (ej != hipSuccess) return ej;
          const int ncg = (int)cdiv(pl.KB, kLjdWaves);
          hipLaunchKernelGGL((diag_accum_ljt<DP>), dim3((unsigned)ljd_grid(pl.nslab, ncg)), dim3(64 * kLjdWaves),
                             SH::lds, stream, reinterpret_cast<const float*>(ws + pl.off_lj),
                             reinterpret_cast<const __bf16*>(ws + pl.off_xsplit),
                             reinterpret_cast<const float2*>(ws + pl.off_zpair), pl.N,
                             reinterpret_cast<const uint2*>(ws + pl.off_ljmask), psel, pl.KB, pl.KP, pl.nslab,
                             pl.rows_per_slab, ncg, pmu, psq, pnk);
        }
      }
      constexpr size_t lds = gather_lds_bytes(DP);
      static_assert(lds <= kMaxLds, "gathering pass 2 exceeds LDS");
      hipError_t e = hipFuncSetAttribute(reinterpret_cast<const void*>(&diag_accum_gather<DP>),
                                         hipFuncAttributeMaxDynamicSharedMemorySize, (int)lds);
      if (e != hipSuccess) return e;
      hipLaunchKernelGGL(diag_accum_gather<DP>, dim3((unsigned)gather_grid(pl.nslab, pl.KB)),
                         dim3(64 * kGatherWaves), lds, stream, X, ldx, pl.N, (int)pl.D,
                         reinterpret_cast<const bf16x8*>(ws + pl.off_mu3),
                         reinterpret_cast<const double*>(ws + pl.off_kcx6lin), pl.KB, pl.KP, rowstat,
                         reinterpret_cast<const uint2*>(ws + pl.off_ljmask), pl.nslab, pl.rows_per_slab,
                         pmu, psq, pnk, dense ? 1 : 0, psel);
      return hipGetLastError();
    }
    if (pl.lj_sparse) {
      // Sparse masks (on average at most 2 needed register-row pairs per tile and
      // block) go to diag_accum_sparse where D is a multiple of 32; both kernels are
      // launched and each returns unless the count selects it.
      int64_t sparse_max = -1;
      if (pl.D == DP) {
        sparse_max = 2 * cdiv(pl.N, 32) * pl.KB;
        const int64_t nw = (int64_t)pl.nslab * pl.rgroups * pl.KB;
        hipLaunchKernelGGL((diag_accum_sparse<DP>), dim3((unsigned)cdiv(nw, kSparseWaves)),
                           dim3(64 * kSparseWaves), 0, stream, X, ldx, pl.N, lj, ljmask, ljcount,
                           sparse_max, pl.KB, pl.KP, rowstat, pl.nslab, pl.rgroups, pl.rows_per_slab,
                           pmu, psq, pnk, dense ? 1 : 0);
      }
      auto launch2 = [&](auto cb_tag, auto nh_tag) -> hipError_t {
        constexpr int CB = decltype(cb_tag)::value;
        constexpr int NH = decltype(nh_tag)::value;
        constexpr size_t lds = accum_lj2_lds_bytes<DP, CB, NH>();
        static_assert(lds <= kMaxLds, "pass-2 tiles exceed LDS");
        if (lds > 65536) {
          hipError_t e = hipFuncSetAttribute(reinterpret_cast<const void*>(&diag_accum_lj2<DP, CB, NH>),
                                             hipFuncAttributeMaxDynamicSharedMemorySize, (int)lds);
          if (e != hipSuccess) return e;
        }
        hipLaunchKernelGGL((diag_accum_lj2<DP, CB, NH>), grid2, dim3(kAccThreads), lds, stream, X, ldx,
                           pl.N, (int)pl.D, lj, ljmask, ljcount, sparse_max, pl.KB, pl.KP, rowstat,
                           pl.nslab, pl.rows_per_slab, pmu, psq, pnk, dense ? 1 : 0);
        return hipGetLastError();
      };
      using J1 = std::integral_constant<int, 1>;
      using J4 = std::integral_constant<int, 4>;
      using J8 = std::integral_constant<int, 8>;
      if constexpr (DP == 128) {
        return pl.cpg == 8 ? launch2(J8{}, J1{}) : launch2(J4{}, std::integral_constant<int, 2>{});
      } else {
        return pl.cpg == 8 ? launch2(J8{}, J1{}) : launch2(J4{}, J1{});
      }
    }
  }
  if (!pl.lj) return hipErrorInvalidValue;   // not a plan of this launcher
  // The stored plan above D = 128: the register-order log-joint tiles of diag_lse_ctile.
  auto launch = [&](auto cb_tag, auto nh_tag) -> hipError_t {
    constexpr int CB = decltype(cb_tag)::value;
    constexpr int NH = decltype(nh_tag)::value;
    constexpr size_t lds = accum_lj_lds_bytes<DP, CB, NH>();
    static_assert(lds <= kMaxLds, "pass-2 tiles exceed LDS");
    if (lds > 65536) {
      hipError_t e = hipFuncSetAttribute(reinterpret_cast<const void*>(&diag_accum_lj<DP, CB, NH>),
                                         hipFuncAttributeMaxDynamicSharedMemorySize, (int)lds);
      if (e != hipSuccess) return e;
    }
    hipLaunchKernelGGL((diag_accum_lj<DP, CB, NH>), grid2, dim3(kAccThreads), lds, stream, X, ldx,
                       pl.N, (int)pl.D, lj, pl.KB, pl.KP, rowstat, pl.nslab, pl.rows_per_slab,
                       pmu, psq, pnk, dense ? 1 : 0);
    return hipGetLastError();
  };
  if constexpr (DP > 128) {
    return launch(std::integral_constant<int, 4>{}, std::integral_constant<int, 2>{});
  } else {
    return hipErrorInvalidValue;   // the stored plan up to D = 128 is the sparse form
  }
}

// ===========================================================================
// bf16 operand contract (FGMM_FLAG_BF16), the arithmetic of the reference's
// diagonal H100 kernels (flash_gmm_diag_h100.py:63-130 pass 1, :159-282 pass 2,
// :317-343 constants), in log2 units:
//   W1_kd = fp32(exp(-lss_kd)) * fp32(0.5 log2 e),   W2_kd = mu_kd * W1_kd      (fp32)
//   c0_k  = (lpi_k - 0.5 (D log 2pi + sum_d lss_kd)) log2 e - 0.5 log2 e sum_d mu_kd^2 e^-lss_kd
//   ll2   = c0_k - bf16(x^2) . bf16(W1_k) + 2 bf16(x) . bf16(W2_k)     (fp32 accumulation)
//   r = 2^(ll2 - logZ2);  Nk = sum r;  mu_acc = bf16(r)^T bf16(x);  rxsq = bf16(r)^T bf16(x^2)
//   sig_acc = rxsq - 2 mu mu_acc + mu^2 Nk   (fp64, in diag_reduce)
// One contraction over F = 2 DP features [x^2 | x] against [-bf16(W1) | 2 bf16(W2)]
// (negation and doubling are exact in bf16) on v_mfma_f32_32x32x16_bf16, 16 features
// per step.  The features form NCH chains (x^2 and x; each split in two above
// D = 128) that are added as (c0 + s_x2) + s_x, so that every kernel configuration
// forms bitwise the same log-joint.  Pass 2 recomputes the contraction (at bf16
// rates that costs less than storing the log-joint).
// ===========================================================================
__host__ __device__ constexpr int bf16_chains(int DP) { return DP > 128 ? 4 : 2; }
// Waves per component block in pass 2 (each owns NCH / NH chains and the matching
// feature columns of r^T [x^2 | x]).
__host__ __device__ constexpr int bf16_parts(int DP) { return DP <= 64 ? 1 : bf16_chains(DP); }
// bf16 per row of the feature tile: an odd multiple of 32 bytes, the stride the
// transposing reads (lds_rows_operand) want.
__host__ __device__ constexpr int bf16_xr_stride(int DP) { return 2 * DP + 16; }

// Partials per row slab and component block in pass 2: one per row group, and with two
// parts per block (D = 96, 128) one per part, since each part then accumulates all
// feature columns for its own 16 of the 32 rows.
__host__ __device__ constexpr int bf16_row_partials(int DP, int CB) {
  return kAccWaves / (CB * bf16_parts(DP)) * (bf16_parts(DP) == 2 ? 2 : 1);
}
__host__ __device__ constexpr size_t bf16_accum_lds_bytes(int DP, int CB) {
  return (size_t)2 * (size_t)(256 / (CB * bf16_parts(DP))) * (size_t)bf16_xr_stride(DP) * 2 +
         (size_t)2 * (256 / (CB * bf16_parts(DP))) * sizeof(float) +
         (bf16_parts(DP) > 1 ? (size_t)kAccWaves * 16 * 64 * sizeof(float) : 0);
}
// The next super-tile waits in registers (float4 per thread) while one is processed.
// The staging each part count leaves room for without spilling to scratch (two parts
// keep a split r and the exchange's sums besides): 8, 4 and 6 float4.
__host__ __device__ constexpr int bf16_stage_cap(int DP) {
  return bf16_parts(DP) == 1 ? 8 : bf16_parts(DP) == 2 ? 4 : 6;
}
__host__ __device__ constexpr bool bf16_accum_fits(int DP, int CB) {
  return bf16_accum_lds_bytes(DP, CB) <= kMaxLds &&
         (256 / (CB * bf16_parts(DP))) * (DP / 4) / kAccThreads <= bf16_stage_cap(DP);
}
// Component blocks per pass-2 workgroup: as many as 8 waves hold (4, or 2 with four
// parts), fewer when K has fewer blocks so that no wave idles, where that shape fits.
__host__ inline int bf16_blocks_per_group(int DP, int KB) {
  int cb = bf16_parts(DP) == 4 ? 2 : 4;
  while (cb > 1 && KB <= cb / 2 && bf16_accum_fits(DP, cb / 2)) cb /= 2;
  return cb;
}

// Prologue: the feature operand in matrix-core order, mu_op[kb][q][lane] = features
// 16q + 8(lane/32) + e of component kb*32 + lane%32 (bf16x8), and c0 per component.
__global__ __launch_bounds__(64) void diag_bf16_prep(const float* __restrict__ mu, int64_t ldmu,
                                                     const float* __restrict__ lss, int64_t ldlss,
                                                     int64_t K, int D, int DP,
                                                     const float* __restrict__ lpi,
                                                     bf16x8* __restrict__ mu_op, float* __restrict__ kc,
                                                     unsigned* __restrict__ ljcount) {
  const int kb = blockIdx.x, lane = threadIdx.x, c = lane & 31, g = lane >> 5;
  if (ljcount && kb == 0) ljcount[lane] = 0u;   // pass 1 counts the needed pairs into these
  const int64_t k = (int64_t)kb * 32 + c;
  const bool valid = k < K;
  const int NCF = DP / 8;
  const float half_log2e = (float)(0.5 * kLog2e);
  for (int q = 0; q < NCF; ++q) {
    bf16x8 v;
#pragma unroll
    for (int e = 0; e < 8; ++e) {
      const int f = 16 * q + 8 * g + e;
      const int d = f < DP ? f : f - DP;
      float val = 0.0f;
      if (valid && d < D) {
        const float w1 = (float)exp(-(double)lss[k * ldlss + d]) * half_log2e;
        val = f < DP ? -(float)(__bf16)w1 : 2.0f * (float)(__bf16)(mu[k * ldmu + d] * w1);
      }
      v[e] = (__bf16)val;   // exact: val is a bf16 value, negated or doubled
    }
    mu_op[((int64_t)kb * NCF + q) * 64 + lane] = v;
  }
  if (g == 0) {
    double C = -INFINITY;
    if (valid) {
      double lsum = 0.0, qs = 0.0;
#pragma unroll 8
      for (int d = 0; d < D; ++d) {
        const double l = (double)lss[k * ldlss + d];
        const double m = (double)mu[k * ldmu + d];
        lsum += l;
        qs = fma(m * m, exp(-l), qs);
      }
      C = ((double)lpi[k] - 0.5 * ((double)D * kLog2Pi + lsum)) * kLog2e - 0.5 * kLog2e * qs;
    }
    kc[k] = (float)C;
  }
}

// The log-joint of a 32 x 32 tile from its NCH chain partials (accumulator layout),
// in the fixed order shared by both passes.
template <int NCH>
__device__ __forceinline__ float bf16_diag_ll(float c0, const float (&s)[NCH]) {
  if constexpr (NCH == 2) {
    return (c0 + s[0]) + s[1];
  } else {
    return (c0 + (s[0] + s[1])) + (s[2] + s[3]);
  }
}

// Pass 1: grid over 128-row tiles, 4 waves of 32 rows.  Each lane rounds its row's
// x and x^2 to bf16 as it loads them; feature blocks of 32 components (and c0)
// stream through an LDS double buffer.  Writes logZ and logZ2 per row.
// With NEED each row's block maximum, rounded up to bf16, stays in LDS, and once
// logZ2 is final the need words and the needed-pair count are written (as for the
// isotropic contract).
template <int DP>
constexpr size_t bf16_lse_lds_bytes() {
  static_assert(bf16_lse_lds_base(DP) == (size_t)2 * (DP / 8) * 64 * sizeof(bf16x8) + (size_t)2 * 32 * sizeof(float),
                "host sizing");
  return bf16_lse_lds_base(DP);
}

template <int DP, bool NEED = false>
__global__ __launch_bounds__(kThreads) void diag_bf16_lse(const float* __restrict__ X, int64_t ldx,
                                                          int64_t N, int D,
                                                          const bf16x8* __restrict__ mu_op,
                                                          const float* __restrict__ kc, int KB,
                                                          float* __restrict__ logZ,
                                                          float* __restrict__ rowstat,
                                                          unsigned* __restrict__ ljmask,
                                                          unsigned* __restrict__ ljcount, int dense) {
  constexpr int NCF = DP / 8;                  // 16-feature chunks
  constexpr int NCH = bf16_chains(DP);
  constexpr int CPC = NCF / NCH;               // chunks per chain
  constexpr int BLK = NCF * 64;                // bf16x8 per 32-component block
  constexpr int LPT = (BLK + kThreads - 1) / kThreads;
  static_assert(NCF % NCH == 0, "chains split the features evenly");

  extern __shared__ __align__(16) unsigned char lds_raw[];
  bf16x8* mu_l = reinterpret_cast<bf16x8*>(lds_raw);                               // [2][BLK]
  float* kc_l = reinterpret_cast<float*>(lds_raw + 2 * BLK * sizeof(bf16x8));      // [2][32]
  unsigned short* rmax_l = reinterpret_cast<unsigned short*>(lds_raw + bf16_lse_lds_bytes<DP>());   // [wave][KB][32]

  const int tid = threadIdx.x, lane = tid & 63, wave = tid >> 6;
  const int c = lane & 31, g = lane >> 5;
  const int64_t tile = (int64_t)blockIdx.x * kWaves + wave;
  const int64_t row = tile * 32 + c;
  const bool valid = row < N;

  bf16x8 st[LPT];
  float kst = 0.0f;
  auto fetch = [&](int kb) {
    const bf16x8* src = mu_op + (int64_t)kb * BLK;
#pragma unroll
    for (int q = 0; q < LPT; ++q)
      if (BLK % kThreads == 0 || q * kThreads + tid < BLK) st[q] = src[q * kThreads + tid];
    if (tid < 32) kst = kc[(int64_t)kb * 32 + tid];
  };
  auto commit = [&](int buf) {
#pragma unroll
    for (int q = 0; q < LPT; ++q)
      if (BLK % kThreads == 0 || q * kThreads + tid < BLK) mu_l[buf * BLK + q * kThreads + tid] = st[q];
    if (tid < 32) kc_l[buf * 32 + tid] = kst;
  };
  fetch(0);

  // This lane's feature chunks: chunk q < NCF/2 is bf16(x^2) of dimensions 16q + 8g ..
  // +7, chunk NCF/2 + q is bf16(x) of the same dimensions.
  bf16x8 xf[NCF];
#pragma unroll
  for (int q = 0; q < NCF / 2; ++q) {
    const int d0 = 16 * q + 8 * g;
    const f32x4 lo = load_row4(X, ldx, row, d0, D, valid), hi = load_row4(X, ldx, row, d0 + 4, D, valid);
    xf[q] = to_bf16x8(lo * lo, hi * hi);
    xf[NCF / 2 + q] = to_bf16x8(lo, hi);
  }
  commit(0);
  lds_barrier();

  float mx = -INFINITY, sm = 0.0f;
  for (int kb = 0; kb < KB; ++kb) {
    const int buf = kb & 1;
    const bool more = kb + 1 < KB;
    if (more) fetch(kb + 1);
    const bf16x8* mp = mu_l + buf * BLK + lane;
    // S^T = W . F^T per chain: lane = row, register i = component acc_row(i, g).
    f32x16 ch[NCH];
#pragma unroll
    for (int h = 0; h < NCH; ++h) ch[h] = zero16();
#pragma unroll
    for (int qq = 0; qq < CPC; ++qq) {
#pragma unroll
      for (int h = 0; h < NCH; ++h) ch[h] = mfma_bf16(mp[(h * CPC + qq) * 64], xf[h * CPC + qq], ch[h]);
    }
    const float* kp = kc_l + buf * 32;
    float ll[16];
    float bm = -INFINITY;
#pragma unroll
    for (int i = 0; i < 16; ++i) {
      float s[NCH];
#pragma unroll
      for (int h = 0; h < NCH; ++h) s[h] = ch[h][i];
      ll[i] = bf16_diag_ll<NCH>(kp[acc_row(i, g)], s);
      bm = fmaxf(bm, ll[i]);
    }
    if constexpr (NEED) rmax_l[(wave * KB + kb) * 32 + c] = bf16_bits_up(lj_row_max(bm));   // both halves: same value
    const float mn = fmaxf(mx, bm);
    const float ms = (mn == -INFINITY) ? 0.0f : mn;
    float a = sm * fast_exp2(mx - ms);
#pragma unroll
    for (int i = 0; i < 16; ++i) a += fast_exp2(ll[i] - ms);
    sm = a;
    mx = mn;
    if (more) commit(buf ^ 1);
    lds_barrier();
  }
  const float mo = __shfl_xor(mx, 32);
  const float so = __shfl_xor(sm, 32);
  const float mn = fmaxf(mx, mo);
  const float ms = (mn == -INFINITY) ? 0.0f : mn;
  const float lz2 = mn + log2f(sm * fast_exp2(mx - ms) + so * fast_exp2(mo - ms));
  if (valid && g == 0) {
    rowstat[row] = lz2;
    if (logZ) logZ[row] = lz2 * (float)kLn2;
  }
  if constexpr (NEED) {
    const unsigned short* rm = rmax_l + wave * KB * 32 + c;
    if (g == 0)
      need_put_masks([&](int kb) { return bf16_bits_to_float(rm[kb * 32]); }, ljmask + tile * KB,
                     ljcount + (tile & 63), KB, c, (double)lz2, valid, dense != 0);
  }
}

// Pass 2: grid over (row slab x group of CB component blocks); 8 waves = CB blocks x
// NH parts x 8/(CB NH) row groups.  Part h of a block holds the feature operand of
// chains [h NCH/NH, (h+1) NCH/NH), recomputes their partial S = F W^T for its 32
// rows, and with NH > 1 the parts meet in LDS and every part forms the same log-joint
// in the shared order.  Each part then accumulates r^T F over its own feature columns
// (x^2 columns into part_sq, x columns into part_mu).  X super-tiles are loaded
// coalesced, squared and rounded once per workgroup into a double-buffered row-major
// feature tile in LDS (x^2 then x): the A operand of S is a 16-byte read per lane, and
// the B operand of r^T F (8 consecutive rows of one feature per lane-half) comes from
// two transposing reads (lds_rows_operand).
template <int DP, int CB, int NH = bf16_parts(DP)>
__global__ __attribute__((amdgpu_flat_work_group_size(kAccThreads, kAccThreads), amdgpu_waves_per_eu(2, 2)))
void diag_bf16_accum(const float* __restrict__ X, int64_t ldx, int64_t N, int D,
                     const bf16x8* __restrict__ mu_op, const float* __restrict__ kc, int KB, int KP,
                     const float* __restrict__ rowstat, int nslab, int64_t rows_per_slab,
                     float* __restrict__ part_mu, float* __restrict__ part_sq,
                     float* __restrict__ part_nk, int dense, const unsigned* __restrict__ needcount,
                     int64_t dense_min) {
  constexpr int F = 2 * DP;                    // features per row
  constexpr int NCF = F / 16;                  // 16-feature chunks
  constexpr int NCH = bf16_chains(DP);
  constexpr int CPC = NCF / NCH;               // chunks per chain
  constexpr int CPW = NCH / NH;                // chains per wave
  // With two parts, part h forms r for the 16 rows of step h and accumulates r^T F
  // over all features for them (r is formed once per element); otherwise each part
  // forms r for all 32 rows and accumulates its own feature columns.
  constexpr bool SPLIT_ROWS = NH == 2;
  constexpr int FW = SPLIT_ROWS ? F : F / NH;  // feature columns per wave
  constexpr int NJ = FW / 32;                  // 32-column tiles of r^T F per wave
  constexpr int RG = kAccWaves / (CB * NH);    // row groups (32 rows each)
  constexpr int TR = 32 * RG;                  // rows per super-tile
  constexpr int XR = bf16_xr_stride(DP);
  constexpr int V4 = DP / 4;
  constexpr int NV = TR * V4;                  // float4 per super-tile
  constexpr int LPT = (NV + kAccThreads - 1) / kAccThreads;
  static_assert(kAccWaves % (CB * NH) == 0 && NCH % NH == 0 &&
                    (NH == 1 || CPW == 1) && FW % 32 == 0 && DP % 32 == 0,
                "even split");

  // With need masks and fewer than dense_min needed pairs diag_bf16_gather runs instead
  // (uniform exit).
  if (needcount && need_total(needcount) < dense_min) return;

  extern __shared__ __align__(16) unsigned char lds_raw[];
  __bf16* xr = reinterpret_cast<__bf16*>(lds_raw);                        // [2][TR][XR]
  float* rs = reinterpret_cast<float*>(xr + 2 * TR * XR);                  // [2][TR]
  float* ex = rs + 2 * TR;                                                 // [8][16][64] (NH > 1)

  const int tid = threadIdx.x, lane = tid & 63, wave = tid >> 6;
  const int c = lane & 31, g = lane >> 5;
  const int cbw = wave % CB, h = (wave / CB) % NH, rg = wave / (CB * NH);
  const int fc = h * (F / NH);                 // first feature of this wave's chains
  const int f0 = SPLIT_ROWS ? 0 : fc;          // first feature of this wave's r^T F columns
  const int slab = blockIdx.x % nslab;
  const int cg = blockIdx.x / nslab;
  const int kb = cg * CB + cbw;
  const bool active = kb < KB;

  const int64_t r_begin = (int64_t)slab * rows_per_slab;
  int64_t r_end = r_begin + rows_per_slab;
  if (r_end > N) r_end = N;
  const int ntiles = r_end > r_begin ? (int)cdiv(r_end - r_begin, TR) : 0;

  // B operand of the recompute (lane = component, features 16q + 8g + e of this
  // wave's chains) and the component's constant.
  bf16x8 mub[CPW * CPC];
#pragma unroll
  for (int q = 0; q < CPW * CPC; ++q) {
    if (active) {
      mub[q] = mu_op[((int64_t)kb * NCF + h * CPW * CPC + q) * 64 + lane];
    } else {
#pragma unroll
      for (int e = 0; e < 8; ++e) mub[q][e] = (__bf16)0.0f;
    }
  }
  const float c0 = active ? kc[(int64_t)kb * 32 + c] : -INFINITY;

  f32x16 acc[NJ];
#pragma unroll
  for (int j = 0; j < NJ; ++j) acc[j] = zero16();
  float nk = 0.0f;

  // X super-tiles go global -> registers -> LDS: tile t + 1 is loaded while tile t
  // is processed.
  f32x4 stage[LPT];
  float rstage = INFINITY;
  const bool full_d = (D == DP);
  // float4 idx of a super-tile <-> (row, 4 dimensions), row-major.
  auto tile_row = [](int idx) { return idx / V4; };
  auto tile_col = [](int idx) { return (idx % V4) * 4; };
  auto fetch = [&](int t) {
    const int64_t row0 = r_begin + (int64_t)t * TR;
    if (full_d && row0 + TR <= r_end) {
      const float* src = X + row0 * ldx;
#pragma unroll
      for (int q = 0; q < LPT; ++q) {
        const int idx = q * kAccThreads + tid;
        if (NV % kAccThreads == 0 || idx < NV)
          stage[q] = *reinterpret_cast<const f32x4*>(src + (int64_t)tile_row(idx) * ldx + tile_col(idx));
      }
    } else {
#pragma unroll
      for (int q = 0; q < LPT; ++q) {
        const int idx = q * kAccThreads + tid;
        const int64_t row = row0 + tile_row(idx);
        if (NV % kAccThreads == 0 || idx < NV)
          stage[q] = load_row4(X, ldx, row, tile_col(idx), D, row < r_end);
      }
    }
    if (tid < TR) {
      const int64_t row = row0 + tid;
      // Rows past the slab get logZ2 = +inf, hence r = 0.
      rstage = (row < r_end) ? rowstat[row] : INFINITY;
    }
  };
  auto commit = [&](int buf) {
    __bf16* dr = xr + buf * TR * XR;
    typedef __bf16 bf16x4 __attribute__((ext_vector_type(4)));
#pragma unroll
    for (int q = 0; q < LPT; ++q) {
      const int idx = q * kAccThreads + tid;
      if (NV % kAccThreads != 0 && idx >= NV) continue;
      const int r = tile_row(idx), d = tile_col(idx);
      const f32x4 v = stage[q];
      const f32x4 v2 = v * v;
      const bf16x4 b = {(__bf16)v.x, (__bf16)v.y, (__bf16)v.z, (__bf16)v.w};
      const bf16x4 b2 = {(__bf16)v2.x, (__bf16)v2.y, (__bf16)v2.z, (__bf16)v2.w};
      *reinterpret_cast<bf16x4*>(dr + r * XR + d) = b2;
      *reinterpret_cast<bf16x4*>(dr + r * XR + DP + d) = b;
    }
    if (tid < TR) rs[buf * TR + tid] = rstage;
  };

  if (ntiles > 0) {
    fetch(0);
    commit(0);
  }
  lds_barrier();

  for (int t = 0; t < ntiles; ++t) {
    const int buf = t & 1;
    const bool more = t + 1 < ntiles;
    if (more) fetch(t + 1);
    // This wave's chain partials of S = F W^T for its 32 rows: lane = component,
    // register i = row acc_row(i, g).
    f32x16 ch[CPW];
#pragma unroll
    for (int u = 0; u < CPW; ++u) ch[u] = zero16();
    if (active) {
      const __bf16* xrow = xr + buf * TR * XR + (rg * 32 + c) * XR + fc + 8 * g;
#pragma unroll
      for (int qq = 0; qq < CPC; ++qq) {
#pragma unroll
        for (int u = 0; u < CPW; ++u)
          ch[u] = mfma_bf16(*reinterpret_cast<const bf16x8*>(xrow + 16 * (u * CPC + qq)), mub[u * CPC + qq],
                            ch[u]);
      }
    }
    // Chain u of register i: this wave's own, or (NH > 1) the one part u of the block
    // wrote to LDS, the parts of a block being waves rg*CB*NH + u*CB + cbw.  The slots
    // hold registers 4q..4q+3 of a lane as one float4, [wave][q][lane].
    const f32x4* s0 = reinterpret_cast<const f32x4*>(ex) + (rg * CB * NH + cbw) * 4 * 64 + lane;
    if constexpr (NH > 1) {
      f32x4* mine = reinterpret_cast<f32x4*>(ex) + wave * 4 * 64 + lane;
#pragma unroll
      for (int q = 0; q < 4; ++q) mine[q * 64] = f32x4{ch[0][4 * q], ch[0][4 * q + 1], ch[0][4 * q + 2], ch[0][4 * q + 3]};
      lds_barrier();
    }
    if constexpr (SPLIT_ROWS) {
      if (active) {
        // Registers 8h .. 8h + 7: rows rg*32 + 16h + 8(q - 2h) + 4g + j.
        const f32x4* rt = reinterpret_cast<const f32x4*>(rs + buf * TR + rg * 32 + 4 * g);
        float r8[8];
#pragma unroll
        for (int qq = 0; qq < 2; ++qq) {
          const int q = 2 * h + qq;
          f32x4 sq[NCH];
#pragma unroll
          for (int u = 0; u < NCH; ++u) sq[u] = s0[(u * CB * 4 + q) * 64];
          const f32x4 lz = rt[2 * q];
#pragma unroll
          for (int j = 0; j < 4; ++j) {
            float sv[NCH];
#pragma unroll
            for (int u = 0; u < NCH; ++u) sv[u] = sq[u][j];
            const float rv = fast_exp2(bf16_diag_ll<NCH>(c0, sv) - lz[j]);
            nk += rv;
            r8[4 * qq + j] = rv;
          }
        }
        const bf16x8 a = acc_to_row_operand(r8);
        const __bf16* xt = xr + buf * TR * XR;
        if (dense || any_nonzero(a)) {
#pragma unroll
          for (int j = 0; j < NJ; ++j)
            acc[j] = mfma_bf16(a, lds_rows_operand(xt, XR, rg * 32 + 16 * h, 32 * j, lane), acc[j]);
        }
      }
    } else if (active) {
      const f32x4* rt = reinterpret_cast<const f32x4*>(rs + buf * TR + rg * 32 + 4 * g);
      float r[16];
#pragma unroll
      for (int q = 0; q < 4; ++q) {
        f32x4 sq[NCH];
#pragma unroll
        for (int u = 0; u < NCH; ++u) {
          if constexpr (NH == 1) {
            sq[u] = f32x4{ch[u][4 * q], ch[u][4 * q + 1], ch[u][4 * q + 2], ch[u][4 * q + 3]};
          } else {
            sq[u] = s0[(u * CB * 4 + q) * 64];
          }
        }
        // Rows acc_row(4q + j, g) = 8q + 4g + j: one float4 of the row state.
        const f32x4 lz = rt[2 * q];
#pragma unroll
        for (int j = 0; j < 4; ++j) {
          float sv[NCH];
#pragma unroll
          for (int u = 0; u < NCH; ++u) sv[u] = sq[u][j];
          const float rv = fast_exp2(bf16_diag_ll<NCH>(c0, sv) - lz[j]);
          if (h == 0) nk += rv;
          r[4 * q + j] = rv;
        }
      }
      bf16x8 a[2];
      acc_to_row_operands(r, a);
      // B operand: rows rg*32 + 16p + 8g + e of feature f0 + 32j + c.
      const __bf16* xt = xr + buf * TR * XR;
#pragma unroll
      for (int p = 0; p < 2; ++p) {
        // A step whose 16 rows x 32 components of bf16(r) are all zero adds nothing.
        if (dense || any_nonzero(a[p])) {
#pragma unroll
          for (int j = 0; j < NJ; ++j)
            acc[j] = mfma_bf16(a[p], lds_rows_operand(xt, XR, rg * 32 + 16 * p, f0 + 32 * j, lane), acc[j]);
        }
      }
    }
    if (more) commit(buf ^ 1);
    lds_barrier();
  }

  if (active) {
    nk += __shfl_xor(nk, 32);
    // Partial index: the row group, and with SPLIT_ROWS the part within it.
    const int rp = SPLIT_ROWS ? rg * NH + h : rg;
    const int64_t kbase = ((int64_t)slab * bf16_row_partials(DP, CB) + rp) * KP + (int64_t)kb * 32;
#pragma unroll
    for (int j = 0; j < NJ; ++j) {
      const int f = f0 + 32 * j;               // a tile lies wholly in x^2 or in x
      float* dst = f < DP ? part_sq + f : part_mu + (f - DP);
#pragma unroll
      for (int i = 0; i < 16; ++i) dst[(kbase + acc_row(i, g)) * DP + c] = acc[j][i];
    }
    if (g == 0 && (SPLIT_ROWS || h == 0)) part_nk[kbase + c] = nk;
  }
}

// Pass 2 of the bf16 contract up to D = 128 where few pairs are needed (pass 1's
// needed-pair count below dense_min; diag_bf16_accum runs otherwise): one wave per
// (row slab, component block), 4 waves of one block on consecutive slabs per
// workgroup, the block's feature operands in LDS.  Each wave queues the rows whose
// need bit is set and per 32 queued rows:
//   - loads them (buffer resource over the slab), forms bf16(x^2) and bf16(x) in the
//     A-operand layout (lane = row) and writes them row-major ([x^2 | x]) to its LDS
//     tile;
//   - S in pass 1's two chains (x^2, then x) and order, the log-joint as
//     (c0 + s_x2) + s_x, so a cleared pair would give r = 0 exactly;
//   - r = 2^(ll2 - logZ2), Nk on the VALU, bf16(r)^T [x^2 | x] on the matrix cores.
// slab counts the partials of diag_bf16_accum's split, so either kernel fills the
// same partial slots.
__host__ __device__ constexpr size_t bf16_gather_lds_bytes(int DP) {
  return (size_t)(DP / 8) * 64 * sizeof(bf16x8)                    // the block's feature operands
         + (size_t)kGatherWaves * 32 * bf16_xr_stride(DP) * 2       // [x^2 | x] tile per wave
         + (size_t)kGatherWaves * 32 * sizeof(float)                // logZ2 per wave
         + (size_t)kGatherWaves * 64 * sizeof(int);                 // row queue per wave
}

template <int DP>
__global__ __attribute__((amdgpu_flat_work_group_size(64 * kGatherWaves, 64 * kGatherWaves),
                          amdgpu_waves_per_eu(gather_waves_per_simd(DP), gather_waves_per_simd(DP))))
void diag_bf16_gather(const float* __restrict__ X, int64_t ldx, int64_t N, int D,
                      const bf16x8* __restrict__ mu_op, const float* __restrict__ kc, int KB, int KP,
                      const float* __restrict__ rowstat, const unsigned* __restrict__ need,
                      const unsigned* __restrict__ needcount, int64_t dense_min, int nslab,
                      int64_t rows_per_slab, float* __restrict__ part_mu, float* __restrict__ part_sq,
                      float* __restrict__ part_nk, int dense) {
  constexpr int NQ = DP / 16;        // 16-dimension chunks (per feature)
  constexpr int NCF = DP / 8;        // 16-feature chunks
  constexpr int NJ = DP / 32;        // 32-column tiles per feature
  constexpr int RS = bf16_xr_stride(DP);
  constexpr int BLK = NCF * 64;      // bf16x8 per component block
  static_assert(DP <= 128 && bf16_chains(DP) == 2, "two chains: x^2, then x");
  if (need_total(needcount) >= dense_min) return;   // diag_bf16_accum runs instead (uniform exit)

  extern __shared__ __align__(16) unsigned char lds_raw[];
  unsigned char* lp = lds_raw;
  bf16x8* mu_l = reinterpret_cast<bf16x8*>(lp);     lp += (size_t)BLK * sizeof(bf16x8);
  __bf16* xt_all = reinterpret_cast<__bf16*>(lp);   lp += (size_t)kGatherWaves * 32 * RS * 2;
  float* rs_all = reinterpret_cast<float*>(lp);     lp += (size_t)kGatherWaves * 32 * sizeof(float);
  int* q_all = reinterpret_cast<int*>(lp);

  const int tid = threadIdx.x, lane = tid & 63;
  const int wave = __builtin_amdgcn_readfirstlane(tid >> 6);
  const int c = lane & 31, g = lane >> 5;
  int sg, kb;
  if (!gather_item(blockIdx.x, gather_groups(nslab), KB, sg, kb)) return;   // uniform over the workgroup
  for (int idx = tid; idx < BLK; idx += 64 * kGatherWaves) mu_l[idx] = mu_op[(int64_t)kb * BLK + idx];
  __syncthreads();
  const int slab = sg * kGatherWaves + wave;
  if (slab >= nslab) return;   // no barrier follows

  __bf16* xt = xt_all + wave * 32 * RS;
  float* rs_l = rs_all + wave * 32;
  int* q_l = q_all + wave * 64;
  const float c0 = kc[(int64_t)kb * 32 + c];

  const int64_t r_begin = (int64_t)slab * rows_per_slab;
  int64_t r_end = r_begin + rows_per_slab;
  if (r_end > N) r_end = N;
  const int64_t t_begin = r_begin / 32, t_end = r_end > r_begin ? cdiv(r_end, 32) : t_begin;

  auto words = [&](int64_t tb) -> unsigned {
    const int64_t t = tb + lane;
    return t < t_end ? need[t * KB + kb] : 0u;
  };
  int64_t tb = t_begin;
  unsigned mword = words(tb), mnext = words(tb + 64);
  int jn = 0;
  int qh = 0, qt = 0;
  auto take = [&](int& e) -> int {
    queue_fill<(DP > 32)>(words, tb, t_begin, t_end, mword, mnext, jn, qt, qh, lane, c, g, q_l);
    const int cnt = qt - qh < 32 ? qt - qh : 32;
    asm volatile("s_waitcnt lgkmcnt(0)" ::: "memory");
    e = c < cnt ? q_l[(qh + c) & 63] : -1;
    qh += cnt;
    return cnt;
  };

  f32x4 raw[2 * NQ];
  float rst;
  const int64_t nrows = r_end > r_begin ? r_end - r_begin : 0;
  const bool xbuf = slab_fits(nrows, ldx);
  const bool xfull = xbuf && D == DP;
  const buf_rsrc xres = slab_rsrc(X, ldx, r_begin, xbuf ? r_begin + nrows : r_begin);
  const buf_rsrc rres = make_rsrc(rowstat + r_begin, (uint32_t)(nrows * sizeof(float)));
  auto issue = [&](int e) __attribute__((always_inline)) {
    const bool ok = e >= 0;
    if (xfull) {
      const int off = buf_off(ok ? (int)((int64_t)e * ldx * (int64_t)sizeof(float)) + 32 * g : kBufOob);
#pragma unroll
      for (int q = 0; q < NQ; ++q) {
        raw[2 * q] = __builtin_bit_cast(f32x4, __builtin_amdgcn_raw_buffer_load_b128(xres, off, 64 * q, 0));
        raw[2 * q + 1] = __builtin_bit_cast(f32x4, __builtin_amdgcn_raw_buffer_load_b128(xres, off, 64 * q + 16, 0));
      }
    } else if (xbuf) {
#pragma unroll
      for (int q = 0; q < NQ; ++q) {
        raw[2 * q] = slab_row4(xres, ldx, e, 16 * q + 8 * g, D, ok);
        raw[2 * q + 1] = slab_row4(xres, ldx, e, 16 * q + 8 * g + 4, D, ok);
      }
    } else {
      const int64_t row = r_begin + (ok ? e : 0);
#pragma unroll
      for (int q = 0; q < NQ; ++q) {
        raw[2 * q] = load_row4(X, ldx, row, 16 * q + 8 * g, D, ok);
        raw[2 * q + 1] = load_row4(X, ldx, row, 16 * q + 8 * g + 4, D, ok);
      }
    }
    const float v = buf_load_f32(rres, buf_off(ok ? e * (int)sizeof(float) : kBufOob));
    rst = ok ? v : INFINITY;   // a row past the queue: logZ2 = +inf, r = 0
  };

  f32x16 acc[2][NJ];   // [x^2 | x] columns
#pragma unroll
  for (int f = 0; f < 2; ++f)
#pragma unroll
    for (int j = 0; j < NJ; ++j) acc[f][j] = zero16();
  float nk = 0.0f;

  int e;
  int cnt = take(e);
  if (cnt > 0) issue(e);
  while (cnt > 0) {
    bf16x8 x2[NQ], x1[NQ];
#pragma unroll
    for (int q = 0; q < NQ; ++q) {
      x2[q] = to_bf16x8(raw[2 * q] * raw[2 * q], raw[2 * q + 1] * raw[2 * q + 1]);
      x1[q] = to_bf16x8(raw[2 * q], raw[2 * q + 1]);
    }
    asm volatile("s_waitcnt lgkmcnt(0)" ::: "memory");   // the previous tile's LDS reads are done
#pragma unroll
    for (int q = 0; q < NQ; ++q) {
      *reinterpret_cast<bf16x8*>(xt + c * RS + 16 * q + 8 * g) = x2[q];
      *reinterpret_cast<bf16x8*>(xt + c * RS + DP + 16 * q + 8 * g) = x1[q];
    }
    if (g == 0) rs_l[c] = rst;
    int en;
    const int cnt_next = take(en);
    if (cnt_next > 0) issue(en);
    asm volatile("s_waitcnt lgkmcnt(0)" ::: "memory");

    // Chains of S = F W^T: lane = component c, register i = row acc_row(i, g).
    f32x16 s0 = zero16(), s1 = zero16();
#pragma unroll
    for (int q = 0; q < NQ; ++q) {
      s0 = mfma_bf16(x2[q], mu_l[q * 64 + lane], s0);
      s1 = mfma_bf16(x1[q], mu_l[(NQ + q) * 64 + lane], s1);
    }
    float r[16];
#pragma unroll
    for (int i = 0; i < 16; ++i) {
      const float sv[2] = {s0[i], s1[i]};
      const float rv = fast_exp2(bf16_diag_ll<2>(c0, sv) - rs_l[acc_row(i, g)]);
      nk += rv;
      r[i] = rv;
    }
    bf16x8 a[2];
    acc_to_row_operands(r, a);
#pragma unroll
    for (int p = 0; p < 2; ++p) {
      // A step whose 16 rows of bf16(r) are all zero adds nothing.
      if (dense || any_nonzero(a[p])) {
#pragma unroll
        for (int f = 0; f < 2; ++f)
#pragma unroll
          for (int j = 0; j < NJ; ++j)
            acc[f][j] = mfma_bf16(a[p], lds_rows_operand(xt, RS, 16 * p, f * DP + 32 * j, lane), acc[f][j]);
      }
    }
    e = en;
    cnt = cnt_next;
  }

  nk += __shfl_xor(nk, 32);
  const int64_t kbase = (int64_t)slab * KP + (int64_t)kb * 32;
#pragma unroll
  for (int j = 0; j < NJ; ++j) {
#pragma unroll
    for (int i = 0; i < 16; ++i) {
      part_sq[(kbase + acc_row(i, g)) * DP + 32 * j + c] = acc[0][j][i];
      part_mu[(kbase + acc_row(i, g)) * DP + 32 * j + c] = acc[1][j][i];
    }
  }
  if (g == 0) part_nk[kbase + c] = nk;
}

template <int DP>
hipError_t launch_bf16(const DiagPlan& pl, const float* X, int64_t ldx, unsigned char* ws,
                       float* logZ, bool run1, bool run2, bool dense, hipStream_t stream) {
  const bf16x8* mu_op = reinterpret_cast<const bf16x8*>(ws + pl.off_musw);
  const float* kc = reinterpret_cast<const float*>(ws + pl.off_kclin);
  float* rowstat = reinterpret_cast<float*>(ws + pl.off_rowstat);
  unsigned* ljmask = reinterpret_cast<unsigned*>(ws + pl.off_ljmask);
  unsigned* ljcount = reinterpret_cast<unsigned*>(ws + pl.off_ljcount);
  if (run1) {
    auto kern = pl.bfneed ? &diag_bf16_lse<DP, (DP <= 128)> : &diag_bf16_lse<DP>;
    const size_t lds1 = bf16_lse_lds_bytes<DP>() + (pl.bfneed ? (size_t)kWaves * 32 * pl.KB * 2 : 0);
    if (lds1 > 65536) {
      hipError_t e = hipFuncSetAttribute(reinterpret_cast<const void*>(kern),
                                         hipFuncAttributeMaxDynamicSharedMemorySize, (int)lds1);
      if (e != hipSuccess) return e;
    }
    hipLaunchKernelGGL(kern, dim3((unsigned)cdiv(pl.N, 32 * kWaves)), dim3(kThreads), lds1,
                       stream, X, ldx, pl.N, (int)pl.D, mu_op, kc, pl.KB, logZ, rowstat, ljmask, ljcount,
                       dense ? 1 : 0);
  }
  if (!run2) return hipGetLastError();
  // With need masks: the gathering pass (one slab per partial of the dense split) when
  // fewer than 3/4 of the (row, block) pairs are needed, else diag_bf16_accum; both are
  // launched and the needed-pair count selects one on the device.
  const int64_t dense_min = cdiv(cdiv(pl.N, 32) * 32 * (int64_t)pl.KB * 3, 4);
  if (pl.bfneed) {
    if constexpr (DP <= 128) {
      constexpr size_t ldsg = bf16_gather_lds_bytes(DP);
      static_assert(ldsg <= kMaxLds, "gathering tiles fit LDS");
      if (ldsg > 65536) {
        hipError_t e = hipFuncSetAttribute(reinterpret_cast<const void*>(&diag_bf16_gather<DP>),
                                           hipFuncAttributeMaxDynamicSharedMemorySize, (int)ldsg);
        if (e != hipSuccess) return e;
      }
      hipLaunchKernelGGL(diag_bf16_gather<DP>, dim3((unsigned)gather_grid(pl.npart, pl.KB)),
                         dim3(64 * kGatherWaves), ldsg, stream, X, ldx, pl.N, (int)pl.D, mu_op, kc, pl.KB, pl.KP,
                         rowstat, ljmask, ljcount, dense_min, pl.npart, (int64_t)round_up(cdiv(pl.N, pl.npart), 32),
                         reinterpret_cast<float*>(ws + pl.off_part_mu), reinterpret_cast<float*>(ws + pl.off_part_sq),
                         reinterpret_cast<float*>(ws + pl.off_part_nk), dense ? 1 : 0);
    }
  }
  auto launch = [&](auto cb_tag) -> hipError_t {
    constexpr int CB = decltype(cb_tag)::value;
    if constexpr (CB * bf16_parts(DP) > kAccWaves) {
      return hipErrorInvalidValue;   // never chosen by the plan
    } else {
      constexpr size_t lds = bf16_accum_lds_bytes(DP, CB);
      if constexpr (!bf16_accum_fits(DP, CB)) {
        return hipErrorInvalidValue;   // never chosen by the plan
      } else {
        if (lds > 65536) {
          hipError_t e = hipFuncSetAttribute(reinterpret_cast<const void*>(&diag_bf16_accum<DP, CB>),
                                             hipFuncAttributeMaxDynamicSharedMemorySize, (int)lds);
          if (e != hipSuccess) return e;
        }
        hipLaunchKernelGGL((diag_bf16_accum<DP, CB>), dim3((unsigned)(pl.nslab * pl.ncg)),
                           dim3(kAccThreads), lds, stream, X, ldx, pl.N, (int)pl.D, mu_op, kc, pl.KB,
                           pl.KP, rowstat, pl.nslab, pl.rows_per_slab,
                           reinterpret_cast<float*>(ws + pl.off_part_mu),
                           reinterpret_cast<float*>(ws + pl.off_part_sq),
                           reinterpret_cast<float*>(ws + pl.off_part_nk), dense ? 1 : 0,
                           pl.bfneed ? ljcount : nullptr, dense_min);
        return hipGetLastError();
      }
    }
  };
  return pl.cpg == 1   ? launch(std::integral_constant<int, 1>{})
         : pl.cpg == 2 ? launch(std::integral_constant<int, 2>{})
                       : launch(std::integral_constant<int, 4>{});
}

// ---------------------------------------------------------------------------
// bf16 operand contract above D = 256 (any D), as for the isotropic model: pass 1
// (diag_bf16_lse_wide) tiles the contraction over components, re-reading each
// wave's 32 rows per tile of kBwCTB component blocks, and accumulates fp32 chains of
// x^2 and x over 256 dimensions at a time into an fp64 sum, to which c0 is added
// in fp64; it stores the fp32 log-joint,
// [32-row tile][KP][32 rows].  Pass 2 (diag_bf16_accum_wide) reads r from it and
// accumulates bf16(r)^T bf16(x) and bf16(r)^T bf16(x^2) per range of kBwDR
// dimensions from bf16 tiles of x and x^2 in LDS.  Calls whose log-joint exceeds
// kMaxLjBytes run as row chunks.
// ---------------------------------------------------------------------------
constexpr int kBwCTB = 2;    // component blocks per pass-1 tile
constexpr int kBwQS = 4;     // 16-dimension chunks per pass-1 stage
constexpr int kBwFlush = 4;  // stages per fp32 chain: its sum then joins an fp64 one
__host__ __device__ constexpr int bw_stage_ops() { return kBwCTB * 2 * kBwQS * 64; }   // bf16x8
__host__ __device__ constexpr size_t bw_lse_lds_bytes() {
  return (size_t)2 * (bw_stage_ops() * sizeof(bf16x8) + kBwCTB * 32 * sizeof(float));
}

__global__ __launch_bounds__(kThreads) void diag_bf16_lse_wide(const float* __restrict__ X, int64_t ldx,
                                                               int64_t N, int D, int DP,
                                                               const bf16x8* __restrict__ mu_op,
                                                               const float* __restrict__ kc, int KB, int KP,
                                                               float* __restrict__ logZ,
                                                               float* __restrict__ rowstat,
                                                               float* __restrict__ lj) {
  constexpr int SO = bw_stage_ops();
  constexpr int LPT = SO / kThreads;
  static_assert(LPT == 2 * kBwCTB && kThreads == kBwQS * 64, "fetch register u = 2 block + feature");
  extern __shared__ __align__(16) unsigned char lds_raw[];
  bf16x8* mu_l = reinterpret_cast<bf16x8*>(lds_raw);                               // [2][SO]
  float* kc_l = reinterpret_cast<float*>(lds_raw + 2 * SO * sizeof(bf16x8));       // [2][CTB * 32]

  const int NQ = DP / 16, NCF = DP / 8, nst = NQ / kBwQS;
  const int ntile = (KB + kBwCTB - 1) / kBwCTB;
  const int tid = threadIdx.x, lane = tid & 63;
  const int wave = __builtin_amdgcn_readfirstlane(tid >> 6);
  const int c = lane & 31, g = lane >> 5;
  const int64_t tile = (int64_t)blockIdx.x * kWaves + wave;
  const int64_t row = tile * 32 + c;
  const bool valid = row < N;
  const int64_t nstage = (int64_t)ntile * nst;

  bf16x8 st[LPT];
  float kst = -INFINITY;
  auto fetch = [&](int64_t s) {
    const int t = (int)(s / nst), qs = (int)(s % nst);
    const int kb0 = t * kBwCTB;
    const int cnt = KB - kb0 < kBwCTB ? KB - kb0 : kBwCTB;
    const int qq = tid >> 6;
#pragma unroll
    for (int u = 0; u < LPT; ++u) {
      const int b = u >> 1, f = u & 1;   // block of the tile; feature (0: x^2, 1: x)
      if (b < cnt) {
        st[u] = mu_op[((int64_t)(kb0 + b) * NCF + f * NQ + kBwQS * qs + qq) * 64 + lane];
      } else {
#pragma unroll
        for (int e = 0; e < 8; ++e) st[u][e] = (__bf16)0.0f;
      }
    }
    if (tid < kBwCTB * 32) kst = tid < cnt * 32 ? kc[(int64_t)kb0 * 32 + tid] : -INFINITY;
  };
  auto commit = [&](int buf) {
#pragma unroll
    for (int u = 0; u < LPT; ++u) mu_l[buf * SO + u * kThreads + tid] = st[u];
    if (tid < kBwCTB * 32) kc_l[buf * kBwCTB * 32 + tid] = kst;
  };
  f32x4 raw[2 * kBwQS];
  auto loadx = [&](int64_t s) {
    const int qs = (int)(s % nst);
#pragma unroll
    for (int qq = 0; qq < kBwQS; ++qq) {
      const int d0 = 16 * (kBwQS * qs + qq) + 8 * g;
      raw[2 * qq] = load_row4(X, ldx, row, d0, D, valid);
      raw[2 * qq + 1] = load_row4(X, ldx, row, d0 + 4, D, valid);
    }
  };

  // Per block two fp32 chains (x^2, x) over kBwFlush stages (256 dimensions), then
  // added to an fp64 sum, so no fp32 chain grows past ~1/4 of its term at D ~ 1000.
  f32x16 acc[kBwCTB][2];
  double sacc[kBwCTB][16];
#pragma unroll
  for (int b = 0; b < kBwCTB; ++b) {
    acc[b][0] = acc[b][1] = zero16();
#pragma unroll
    for (int i = 0; i < 16; ++i) sacc[b][i] = 0.0;
  }
  float mx = -INFINITY, sm = 0.0f;
  float* ljr = lj + tile * (int64_t)KP * 32 + c;

  if (nstage > 0) {
    fetch(0);
    loadx(0);
    commit(0);
  }
  __syncthreads();
  for (int64_t s = 0; s < nstage; ++s) {
    const int buf = (int)(s & 1);
    const bool more = s + 1 < nstage;
    const int t = (int)(s / nst), qs = (int)(s % nst);
    const int kb0 = t * kBwCTB;
    const int cnt = KB - kb0 < kBwCTB ? KB - kb0 : kBwCTB;
    bf16x8 x2[kBwQS], x1[kBwQS];
#pragma unroll
    for (int qq = 0; qq < kBwQS; ++qq) {
      x2[qq] = to_bf16x8(raw[2 * qq] * raw[2 * qq], raw[2 * qq + 1] * raw[2 * qq + 1]);
      x1[qq] = to_bf16x8(raw[2 * qq], raw[2 * qq + 1]);
    }
    if (more) {
      fetch(s + 1);
      loadx(s + 1);
    }
    const bf16x8* mp = mu_l + buf * SO + lane;
#pragma unroll
    for (int b = 0; b < kBwCTB; ++b) {
      if (b < cnt) {
#pragma unroll
        for (int qq = 0; qq < kBwQS; ++qq) {
          const bf16x8 w2 = mp[((2 * b) * kBwQS + qq) * 64];
          const bf16x8 w1 = mp[((2 * b + 1) * kBwQS + qq) * 64];
          acc[b][0] = mfma_bf16(w2, x2[qq], acc[b][0]);
          acc[b][1] = mfma_bf16(w1, x1[qq], acc[b][1]);
        }
      }
    }
    if ((qs + 1) % kBwFlush == 0 || qs == nst - 1) {
#pragma unroll
      for (int b = 0; b < kBwCTB; ++b) {
#pragma unroll
        for (int i = 0; i < 16; ++i) sacc[b][i] += (double)acc[b][0][i] + (double)acc[b][1][i];
        acc[b][0] = acc[b][1] = zero16();
      }
    }
    if (qs == nst - 1) {   // the tile's blocks are complete: lane = row, register i = component
      const float* kp = kc_l + buf * kBwCTB * 32;
      float bm = -INFINITY;
      float ll[kBwCTB][16];
#pragma unroll
      for (int b = 0; b < kBwCTB; ++b) {
#pragma unroll
        for (int i = 0; i < 16; ++i) {
          // c0 + the fp64 sum of the chains (each term ~4 D log2 units on clustered
          // data), rounded once.
          ll[b][i] = (float)((double)kp[b * 32 + acc_row(i, g)] + sacc[b][i]);
          sacc[b][i] = 0.0;
          if (b < cnt) {
            if (valid) ljr[((int64_t)(kb0 + b) * 32 + acc_row(i, g)) * 32] = ll[b][i];
            bm = fmaxf(bm, ll[b][i]);
          }
        }
      }
      const float mn = fmaxf(mx, bm);
      const float ms = (mn == -INFINITY) ? 0.0f : mn;
      float a = sm * fast_exp2(mx - ms);
#pragma unroll
      for (int b = 0; b < kBwCTB; ++b) {
        if (b < cnt) {
#pragma unroll
          for (int i = 0; i < 16; ++i) a += fast_exp2(ll[b][i] - ms);
        }
      }
      sm = a;
      mx = mn;
    }
    if (more) commit(buf ^ 1);
    lds_barrier();
  }
  const float mo = __shfl_xor(mx, 32);
  const float so = __shfl_xor(sm, 32);
  const float mn = fmaxf(mx, mo);
  const float ms = (mn == -INFINITY) ? 0.0f : mn;
  const float lz2 = mn + log2f(sm * fast_exp2(mx - ms) + so * fast_exp2(mo - ms));
  if (valid && g == 0) {
    rowstat[row] = lz2;
    if (logZ) logZ[row] = lz2 * (float)kLn2;
  }
}

// Pass 2: one workgroup per (row slab, group of kBwCB component blocks, range of
// kBwDR dimensions); wave u owns block cg kBwCB + u and every column of the range in
// both features.  Per 32-row tile the workgroup stages bf16(x) and bf16(x^2) of the
// rows' range (row-major, stride kBwDR + 16) and their logZ2; each lane forms r for
// its component and the 8 rows of each 16-row step its half-wave supplies (the A
// layout of bf16(r)^T F).  The waves of range 0 also sum Nk.
__host__ __device__ constexpr int bw_xr() { return kBwDR + 16; }
__host__ __device__ constexpr size_t bw_accum_lds_bytes() {
  return (size_t)2 * 2 * 32 * bw_xr() * sizeof(__bf16) + (size_t)2 * 32 * sizeof(float);
}

__global__ __attribute__((amdgpu_flat_work_group_size(64 * kBwCB, 64 * kBwCB), amdgpu_waves_per_eu(2, 2)))
void diag_bf16_accum_wide(const float* __restrict__ X, int64_t ldx, int64_t N, int D, int DP, int KB, int KP,
                          const float* __restrict__ rowstat, const float* __restrict__ lj, int nslab,
                          int64_t rows_per_slab, int ncg, int ndr, float* __restrict__ part_mu,
                          float* __restrict__ part_sq, float* __restrict__ part_nk, int dense) {
  constexpr int T = 64 * kBwCB;
  constexpr int XR = bw_xr();
  constexpr int NJ = kBwDR / 32;
  constexpr int LPT = 32 * (kBwDR / 4) / T;   // float4 of the X tile per thread
  static_assert(LPT * T == 32 * kBwDR / 4, "even split");
  extern __shared__ __align__(16) unsigned char lds_raw[];
  __bf16* xr = reinterpret_cast<__bf16*>(lds_raw);                      // [2][2][32][XR]: x^2, then x
  float* rs = reinterpret_cast<float*>(xr + 2 * 2 * 32 * XR);            // [2][32]

  const int tid = threadIdx.x, lane = tid & 63;
  const int wave = __builtin_amdgcn_readfirstlane(tid >> 6);
  const int c = lane & 31, g = lane >> 5;
  const int dr = (int)(blockIdx.x % ndr);
  const int64_t rest = blockIdx.x / ndr;
  const int cg = (int)(rest % ncg);
  const int slab = (int)(rest / ncg);
  const int kb = cg * kBwCB + wave;
  const bool active = kb < KB;
  const bool stats = active && dr == 0;
  const int col0 = dr * kBwDR;
  const int64_t r_begin = (int64_t)slab * rows_per_slab;
  int64_t r_end = r_begin + rows_per_slab;
  if (r_end > N) r_end = N;
  const int ntiles = r_end > r_begin ? (int)cdiv(r_end - r_begin, 32) : 0;
  const int64_t comp = (int64_t)kb * 32 + c;

  f32x4 stage[LPT];
  float rstage = INFINITY;
  auto fetch = [&](int t) {
    const int64_t row0 = r_begin + (int64_t)t * 32;
#pragma unroll
    for (int q = 0; q < LPT; ++q) {
      const int idx = q * T + tid;
      const int64_t rw = row0 + idx / (kBwDR / 4);
      stage[q] = load_row4(X, ldx, rw, col0 + (idx % (kBwDR / 4)) * 4, D, rw < r_end);
    }
    if (tid < 32) rstage = row0 + tid < r_end ? rowstat[row0 + tid] : INFINITY;
  };
  auto commit = [&](int buf) {
    __bf16* dst = xr + buf * 2 * 32 * XR;
    typedef __bf16 bf16x4 __attribute__((ext_vector_type(4)));
#pragma unroll
    for (int q = 0; q < LPT; ++q) {
      const int idx = q * T + tid;
      const f32x4 v = stage[q];
      const int o = (idx / (kBwDR / 4)) * XR + (idx % (kBwDR / 4)) * 4;
      *reinterpret_cast<bf16x4*>(dst + o) = bf16x4{(__bf16)(v.x * v.x), (__bf16)(v.y * v.y), (__bf16)(v.z * v.z),
                                                   (__bf16)(v.w * v.w)};
      *reinterpret_cast<bf16x4*>(dst + 32 * XR + o) = bf16x4{(__bf16)v.x, (__bf16)v.y, (__bf16)v.z, (__bf16)v.w};
    }
    if (tid < 32) rs[buf * 32 + tid] = rstage;
  };

  f32x16 acc[2][NJ];
#pragma unroll
  for (int f = 0; f < 2; ++f)
#pragma unroll
    for (int j = 0; j < NJ; ++j) acc[f][j] = zero16();
  float nk = 0.0f;
  if (ntiles > 0) {
    fetch(0);
    commit(0);
  }
  lds_barrier();
  for (int t = 0; t < ntiles; ++t) {
    const int buf = t & 1;
    const bool more = t + 1 < ntiles;
    if (more) fetch(t + 1);
    if (active) {
      const int64_t row0 = r_begin + (int64_t)t * 32;
      const float* lrow = lj + (((row0 >> 5) * KP) + comp) * 32;
      const float* rt = rs + buf * 32;
      bf16x8 a[2];
#pragma unroll
      for (int p = 0; p < 2; ++p) {
        const f32x4 l0 = *reinterpret_cast<const f32x4*>(lrow + 16 * p + 8 * g);
        const f32x4 l1 = *reinterpret_cast<const f32x4*>(lrow + 16 * p + 8 * g + 4);
        const float lv[8] = {l0.x, l0.y, l0.z, l0.w, l1.x, l1.y, l1.z, l1.w};
        float r8[8];
#pragma unroll
        for (int e = 0; e < 8; ++e) {
          const int rr = 16 * p + 8 * g + e;
          // rows past N hold no log-joint
          const float rv = row0 + rr < r_end ? fast_exp2(lv[e] - rt[rr]) : 0.0f;
          r8[e] = rv;
          if (stats) nk += rv;
        }
        a[p] = to_bf16x8(f32x4{r8[0], r8[1], r8[2], r8[3]}, f32x4{r8[4], r8[5], r8[6], r8[7]});
      }
      const __bf16* xt = xr + buf * 2 * 32 * XR;
#pragma unroll
      for (int p = 0; p < 2; ++p) {
        // A step whose 16 rows x 32 components of bf16(r) are all zero adds nothing.
        if (dense || any_nonzero(a[p])) {
#pragma unroll
          for (int f = 0; f < 2; ++f)
#pragma unroll
            for (int j = 0; j < NJ; ++j)
              acc[f][j] = mfma_bf16(a[p], lds_rows_operand(xt + f * 32 * XR, XR, 16 * p, 32 * j, lane), acc[f][j]);
        }
      }
    }
    if (more) commit(buf ^ 1);
    lds_barrier();
  }
  if (!active) return;
  const int64_t kbase = (int64_t)slab * KP + (int64_t)kb * 32;
#pragma unroll
  for (int j = 0; j < NJ; ++j) {
    const int col = col0 + 32 * j + c;
    if (col < DP) {
#pragma unroll
      for (int i = 0; i < 16; ++i) {
        part_sq[(kbase + acc_row(i, g)) * DP + col] = acc[0][j][i];
        part_mu[(kbase + acc_row(i, g)) * DP + col] = acc[1][j][i];
      }
    }
  }
  if (dr == 0) {
    nk += __shfl_xor(nk, 32);
    if (g == 0) part_nk[kbase + c] = nk;
  }
}

hipError_t launch_bf16_wide(const DiagPlan& pl, const float* X, int64_t ldx, unsigned char* ws, float* logZ,
                            bool run1, bool run2, bool dense, hipStream_t stream) {
  const bf16x8* mu_op = reinterpret_cast<const bf16x8*>(ws + pl.off_musw);
  const float* kc = reinterpret_cast<const float*>(ws + pl.off_kclin);
  float* rowstat = reinterpret_cast<float*>(ws + pl.off_rowstat);
  float* lj = reinterpret_cast<float*>(ws + pl.off_lj);
  if (run1) {
    constexpr size_t lds1 = bw_lse_lds_bytes();
    static_assert(lds1 <= 65536, "pass-1 stages fit the default LDS allocation");
    hipLaunchKernelGGL(diag_bf16_lse_wide, dim3((unsigned)cdiv(pl.N, 32 * kWaves)), dim3(kThreads), lds1, stream,
                       X, ldx, pl.N, (int)pl.D, pl.DP, mu_op, kc, pl.KB, pl.KP, logZ, rowstat, lj);
  }
  if (!run2) return hipGetLastError();
  constexpr size_t lds2 = bw_accum_lds_bytes();
  static_assert(lds2 <= 65536, "pass-2 tiles fit the default LDS allocation");
  hipLaunchKernelGGL(diag_bf16_accum_wide, dim3((unsigned)((int64_t)pl.nslab * pl.ncg * pl.ndr)), dim3(64 * kBwCB),
                     lds2, stream, X, ldx, pl.N, (int)pl.D, pl.DP, pl.KB, pl.KP, rowstat, lj, pl.nslab,
                     pl.rows_per_slab, pl.ncg, pl.ndr, reinterpret_cast<float*>(ws + pl.off_part_mu),
                     reinterpret_cast<float*>(ws + pl.off_part_sq), reinterpret_cast<float*>(ws + pl.off_part_nk),
                     dense ? 1 : 0);
  return hipGetLastError();
}

}  // namespace
}  // namespace fgmm

using namespace fgmm;

namespace {
// Rows per call of the bf16 contract above D = 256, whose log-joint must fit
// kMaxLjBytes: a multiple of 128 rows.  Larger calls run in chunks of this many rows.
int64_t diag_bw_chunk_rows(int64_t K) {
  const int64_t KP = round_up(K < 1 ? 1 : K, 32);
  return (int64_t)(kMaxLjBytes / ((size_t)KP * 32 * sizeof(float))) / 4 * 4 * 32;
}
bool diag_bw_call(int64_t D, unsigned flags) {
  return (flags & FGMM_FLAG_BF16) != 0 && diag_bf16_wide(diag_padded_dim(D));
}
}  // namespace

extern "C" size_t fgmm_diag_workspace_bytes(int64_t N, int64_t K, int64_t D) {
  if (N < 0 || K < 0 || D < 1) return 0;
  return make_plan(N, K, D, false).total;
}

extern "C" size_t fgmm_diag_workspace_bytes_ex(int64_t N, int64_t K, int64_t D, unsigned flags) {
  if (N < 0 || K < 0 || D < 1) return 0;
  const int64_t rows = diag_bw_call(D, flags) ? std::min(N, diag_bw_chunk_rows(K)) : N;
  return make_plan(rows, K, D, wants_stored_lj(flags), (flags & FGMM_FLAG_BF16) != 0, wants_auto_lj(flags)).total;
}

extern "C" int fgmm_diag_estep_f32(const float* X, int64_t ldx, int64_t N, int64_t D, const float* mu,
                                   int64_t ldmu, int64_t K, const float* log_sigma_sq, int64_t ldlss,
                                   const float* log_pi, float* logZ, float* Nk, float* mu_acc,
                                   float* sig_acc, void* workspace, size_t workspace_bytes,
                                   unsigned flags, void* stream_) {
  hipStream_t stream = reinterpret_cast<hipStream_t>(stream_);
  const bool want_logz = !(flags & FGMM_FLAG_NO_LOGZ);
  const bool accumulate = (flags & FGMM_FLAG_ACCUMULATE) != 0;
  const bool dense = (flags & FGMM_FLAG_DENSE) != 0;
  if (N < 0 || K < 0 || D < 1) return FGMM_ERR_INVALID_ARG;
  if (N > 0 && (X == nullptr || ldx < round_up(D, 4) || (ldx % 4) != 0 ||
                (reinterpret_cast<uintptr_t>(X) & 15) != 0))
    return FGMM_ERR_INVALID_ARG;
  if (N > 0 && want_logz && logZ == nullptr) return FGMM_ERR_INVALID_ARG;
  if (K > 0 && (mu == nullptr || ldmu < D || log_sigma_sq == nullptr || ldlss < D ||
                log_pi == nullptr || Nk == nullptr || mu_acc == nullptr || sig_acc == nullptr))
    return FGMM_ERR_INVALID_ARG;
  if (N > kMaxRows || K > (int64_t)1 << 24) return FGMM_ERR_UNSUPPORTED;
  const bool bf16 = (flags & FGMM_FLAG_BF16) != 0;
  if (diag_bw_call(D, flags) && K > 0 && N > diag_bw_chunk_rows(K)) {
    // The bf16 contract above D = 256 stores the log-joint, at most kMaxLjBytes per
    // call: larger N runs as consecutive row chunks on one workspace, each chunk after
    // the first adding its statistics to the outputs.  A phase split cannot span them.
    if (flags & (FGMM_FLAG_PHASE1 | FGMM_FLAG_PHASE2)) return FGMM_ERR_UNSUPPORTED;
    const int64_t rows = diag_bw_chunk_rows(K);
    for (int64_t r0 = 0; r0 < N; r0 += rows) {
      const int64_t n = std::min(rows, N - r0);
      const unsigned f = r0 == 0 ? flags : (flags | FGMM_FLAG_ACCUMULATE);
      const int st = fgmm_diag_estep_f32(X + r0 * ldx, ldx, n, D, mu, ldmu, K, log_sigma_sq, ldlss, log_pi,
                                         logZ ? logZ + r0 : nullptr, Nk, mu_acc, sig_acc, workspace,
                                         workspace_bytes, f, stream_);
      if (st != FGMM_OK) return st;
    }
    return FGMM_OK;
  }
  // The stored-log-joint pass 2 addresses X tiles with 32-bit buffer offsets (row
  // stride at most kMaxBufLdx floats); wider strides recompute, which needs less
  // workspace.
  const DiagPlan pl = make_plan(N, K, D, wants_stored_lj(flags) && ldx <= kMaxBufLdx, bf16, wants_auto_lj(flags));
  if (workspace_bytes < pl.total || (pl.total > 0 && workspace == nullptr)) return FGMM_ERR_WORKSPACE;
  if (!want_logz) logZ = nullptr;
  unsigned char* ws = static_cast<unsigned char*>(workspace);
  const bool sel1 = (flags & FGMM_FLAG_PHASE1) != 0, sel2 = (flags & FGMM_FLAG_PHASE2) != 0;
  const bool run1 = sel1 || !sel2, run2 = sel2 || !sel1;

  if (K == 0) {
    if (N > 0 && logZ)
      hipLaunchKernelGGL(diag_fill, dim3((unsigned)cdiv(N, 256)), dim3(256), 0, stream, logZ, N,
                         -INFINITY);
    return hipGetLastError() == hipSuccess ? FGMM_OK : FGMM_ERR_HIP;
  }
  if (run1 && bf16)
    hipLaunchKernelGGL(diag_bf16_prep, dim3(pl.KB), dim3(64), 0, stream, mu, ldmu, log_sigma_sq, ldlss, K,
                       (int)D, pl.DP, log_pi, reinterpret_cast<bf16x8*>(ws + pl.off_musw),
                       reinterpret_cast<float*>(ws + pl.off_kclin),
                       pl.bfneed ? reinterpret_cast<unsigned*>(ws + pl.off_ljcount) : nullptr);
  else if (run1)
    hipLaunchKernelGGL(diag_x6_prep, dim3(pl.KB), dim3(64), 0, stream, mu, ldmu, log_sigma_sq, ldlss, K,
                       (int)D, pl.DP, log_pi, reinterpret_cast<bf16x8*>(ws + pl.off_mu3),
                       reinterpret_cast<double*>(ws + pl.off_kcx6),
                       reinterpret_cast<double*>(ws + pl.off_kcx6lin),
                       pl.lj_sparse ? reinterpret_cast<unsigned*>(ws + pl.off_ljcount) : nullptr);
  if (N > 0) {
    auto run = [&](auto dp_tag) -> hipError_t {
      constexpr int DP = decltype(dp_tag)::value;
      return bf16 ? launch_bf16<DP>(pl, X, ldx, ws, logZ, run1, run2, dense, stream)
                  : launch_passes<DP>(pl, X, ldx, ws, logZ, run1, run2, dense, stream);
    };
    hipError_t e = hipSuccess;
    if (pl.bfw) {
      e = launch_bf16_wide(pl, X, ldx, ws, logZ, run1, run2, dense, stream);
    } else if (pl.ctile) {
      e = launch_ctile(pl, X, ldx, ws, logZ, run1, run2, dense, stream);
      if (e == hipSuccess && pl.lj && run2) {
        if (pl.DP == 192) e = launch_passes<192>(pl, X, ldx, ws, logZ, false, true, dense, stream);
        else if (pl.DP == 256) e = launch_passes<256>(pl, X, ldx, ws, logZ, false, true, dense, stream);
        else return FGMM_ERR_UNSUPPORTED;
      }
    } else switch (pl.DP) {
      case 32: e = run(std::integral_constant<int, 32>{}); break;
      case 64: e = run(std::integral_constant<int, 64>{}); break;
      case 96: e = run(std::integral_constant<int, 96>{}); break;
      case 128: e = run(std::integral_constant<int, 128>{}); break;
      case 192: e = run(std::integral_constant<int, 192>{}); break;
      case 256: e = run(std::integral_constant<int, 256>{}); break;
      default: return FGMM_ERR_UNSUPPORTED;
    }
    if (e != hipSuccess) return FGMM_ERR_HIP;
  }
  if (!run2) return hipGetLastError() == hipSuccess ? FGMM_OK : FGMM_ERR_HIP;
  if ((flags & FGMM_FLAG_ATOMIC_REDUCE) && !bf16) {
    if (!accumulate) {
      hipLaunchKernelGGL(diag_fill, dim3((unsigned)cdiv(K, 256)), dim3(256), 0, stream, Nk, K, 0.0f);
      hipLaunchKernelGGL(diag_fill, dim3((unsigned)cdiv(K * D, 256)), dim3(256), 0, stream, mu_acc, K * D, 0.0f);
      hipLaunchKernelGGL(diag_fill, dim3((unsigned)cdiv(K * D, 256)), dim3(256), 0, stream, sig_acc, K * D, 0.0f);
    }
    if (pl.npart > 0)
      hipLaunchKernelGGL(diag_reduce_atomic, dim3((unsigned)cdiv(K * D, 256), (unsigned)pl.npart), dim3(256), 0,
                         stream, reinterpret_cast<const float*>(ws + pl.off_part_mu),
                         reinterpret_cast<const float*>(ws + pl.off_part_sq),
                         reinterpret_cast<const float*>(ws + pl.off_part_nk), pl.KP, pl.DP, K, (int)D, mu,
                         ldmu, Nk, mu_acc, sig_acc);
    return hipGetLastError() == hipSuccess ? FGMM_OK : FGMM_ERR_HIP;
  }
  const bool wide = pl.npart >= kWideReduce;
  hipLaunchKernelGGL(wide ? diag_reduce<true> : diag_reduce<false>,
                     dim3((unsigned)(wide ? cdiv(K * D, 4) : cdiv(K * D, 256))), dim3(256), 0, stream,
                     reinterpret_cast<const float*>(ws + pl.off_part_mu),
                     reinterpret_cast<const float*>(ws + pl.off_part_sq),
                     reinterpret_cast<const float*>(ws + pl.off_part_nk), pl.npart, pl.KP, pl.DP, K,
                     (int)D, mu, ldmu, Nk, mu_acc, sig_acc, accumulate ? 1 : 0);
  return hipGetLastError() == hipSuccess ? FGMM_OK : FGMM_ERR_HIP;
}
