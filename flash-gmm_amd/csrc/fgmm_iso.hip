// Isotropic (spherical-covariance) GMM E-step for gfx950.
//
// Math (reference: flash_gmm.py:84-103 pass 1, :141-166 pass 2), in log2 units:
//   b_k   = 0.5 * exp(-lss_k) * log2(e)
//   C_k   = (lpi_k - 0.5*D*(log(2pi) + lss_k)) * log2(e) - b_k * ||mu_k||^2
//   ll2_nk = C_k - b_k * (||x_n||^2 - 2 x_n.mu_k)
//   logZ2_n = log2 sum_k 2^ll2_nk ;  r_nk = 2^(ll2_nk - logZ2_n)
//   Nk_k = sum_n r_nk ; mu_acc_k = sum_n r_nk x_n ; sig_acc_k = sum_n r_nk ||x_n - mu_k||^2
//
// Kernels, all launched on the caller's stream:
//   iso_prep    O(K*D): per-component constants (fp64), mu as three-way bf16 splits
//               with per-chunk centring offsets in matrix-core operand order, and
//               the needed-pair counters zeroed.
//   iso_lse_pipe
//               pass 1 of the default plan up to D = 128: iso_lse's arithmetic in an
//               8-wave workgroup whose two waves per SIMD run a block's contraction
//               and the previous block's epilogue in opposite orders (ping-pong), so
//               one wave's VALU work runs under the other's matrix steps.
//   iso_lse     pass 1 of the stored plan up to D = 128 (two waves per SIMD), and at
//               D = 192 and 256 on the default plan (one wave per SIMD, four chains in
//               iso_lse_ctile's order), grid over row tiles.  Each wave keeps 32 rows
//               of X resident in registers as bf16 splits and streams mu in blocks
//               of 32 components through LDS; the cross term is the centred
//               split-bf16 contraction (x6c_tile, lane = row, register = component)
//               and the log-sum-exp is an online max/sum in registers.  Writes logZ
//               and per-row (||x||^2, logZ2) in fp64 and, after the last block, the
//               need masks (one bit per row and 32-component block: set where the
//               row's responsibility in the block can be nonzero) and their count;
//               with the stored log-joint also its rows (row-major tiles) and each
//               row's block maximum.
//   iso_lse_ctile
//               pass 1 above D = 128 (any D; the default plan uses it above 256): the
//               contraction tiled over components (64 or 128 per tile) as well as
//               rows, the rows' chunks re-read and split per component tile, four
//               accumulation chains.  Same outputs.
//   iso_accum_gather / iso_accum_tiles / iso_accum_tiles2
//               pass 2 of the default plan up to D = 128: the log-joint of the
//               needed (row, block) pairs recomputed bit for bit as pass 1 forms it,
//               r = 2^(ll2 - logZ2), r^T X as split-bf16 products on the matrix cores,
//               Nk and sig_acc on the VALU, one partial per (slab, component).  The
//               gathering kernel queues the needed rows of each slab; the tile
//               kernels (most pairs needed) visit every row, at D = 96 and 128 with
//               two waves per block, one accumulation chain each.  The needed-pair
//               count selects one of them on the device.
//   iso_accum_drange
//               pass 2 of the default plan above D = 128: per (slab, block, range of
//               up to 1024 dimensions) four waves share the queued rows, each forming
//               one chain of the contraction and a quarter of r^T X.
//   iso_accum_sparse / iso_accum_lj
//               pass 2 of the stored plan (FGMM_FLAG_STORE_LOGJOINT, D <= 256): the
//               needed rows of the stored log-joint instead of a recomputation.
//   iso_reduce  fixed-order fp64 sum of the slab partials (deterministic), or
//               the atomic variant selected by FGMM_FLAG_ATOMIC_REDUCE.
//   iso_bf16_*  the bf16 operand contract (FGMM_FLAG_BF16).
//
// Accuracy: the split-bf16 contraction keeps each 16-dimension chunk's result small
// (centred on the chunk's ||mu_q||^2) and sums the chunks in fp32 chains (two up to
// D = 128, four above), then combines them with the fp64 ||x||^2 and constants.
// A single fp32 chain of fp32 matrix steps over D=128 would leave ~3e-4 absolute
// error in logZ on clustered data.

#include "fgmm_common.hpp"

#include <float.h>
#include <math.h>

#include <algorithm>
#include <type_traits>

namespace fgmm {
namespace {

constexpr int kWaves = 4;        // waves per workgroup
constexpr int kThreads = 64 * kWaves;

// Per-row state of pass 2 in LDS: logZ2 in fp64 and ||x||^2 in fp32.
struct __align__(16) RowStat {
  double q;
  float h;
  float pad;
};
constexpr int kAccWaves = 8;   // pass-2 LDS variant: waves per workgroup
constexpr int kAccThreads = 64 * kAccWaves;


constexpr size_t kMaxLds = 160 * 1024;

// Above D = 128 the default plan tiles pass 1 over components as well
// (iso_lse_ctile) and splits pass 2 over dimension ranges (iso_accum_drange); D is
// padded to a multiple of 64 there, so each of the four accumulation chains gets
// the same number of 16-dimension chunks.
constexpr int kCtWaves = 4;                               // waves per workgroup, one per SIMD
constexpr int kGatherWaves = 4;                           // waves (row slabs) per gathering workgroup
constexpr int kCtChains = 4;                              // accumulation chains (chunk q -> q % 4)
constexpr int kDrange = 1024;                             // dimensions of r^T X per pass-2 workgroup
constexpr int kDrTiles = kDrange / 32 / kCtWaves;         // 32-column tiles per pass-2 wave

// Component blocks per pass-1 tile: 2 up to D = 512 (two waves per SIMD, which the
// 128 accumulator registers of 2 blocks x 4 chains allow), 4 above (one wave per SIMD;
// the rows are re-read once per component tile, and at large D the reads of the
// narrower tile cost more than the second wave gains).
__host__ __device__ constexpr int ctile_blocks(int DP) { return DP <= 512 ? 2 : 4; }
__host__ __device__ constexpr int ctile_stage_ops(int CTB) { return CTB * 2 * 4 * 64; }   // bf16x8 per two-chunk stage
__host__ __device__ constexpr size_t lse_ctile_base(int CTB) {
  return (size_t)2 * ctile_stage_ops(CTB) * sizeof(bf16x8) + (size_t)2 * CTB * 32 * sizeof(double2);
}
// Component blocks whose need bounds (bf16, 32 rows per wave) fit beside the stages.
__host__ __device__ constexpr int ctile_need_exact_cap(int CTB) {
  return (int)((kMaxLds - lse_ctile_base(CTB)) / (kCtWaves * 32 * 2));
}
__host__ __device__ constexpr int drange_rs(int DR) { return DR + 16; }   // bf16 row stride of the X tile
__host__ __device__ constexpr size_t accum_drange_lds_bytes(int DR) {
  return (size_t)2 * 32 * drange_rs(DR) * 2                 // x1, x2 of 32 rows
         + (size_t)kCtWaves * 16 * 64 * sizeof(float)        // the four chains of S
         + (size_t)32 * sizeof(double2)                      // row state
         + (size_t)kCtWaves * 64 * sizeof(int);              // row queue per wave
}

__host__ inline int iso_padded_dim(int64_t D) {
  return D <= 128 ? (int)round_up(D < 1 ? 1 : D, 32) : (int)round_up(D, 64);
}

struct IsoPlan {
  int64_t N, K, D;
  int DP;       // D padded to a multiple of 32 (of 64 above 128)
  int KB;       // 32-component blocks
  int KP;       // K padded to a multiple of 32
  int cpg;      // component blocks per pass-2 workgroup
  int ncg;      // groups of cpg component blocks (pass 2)
  int nslab;    // row slabs (pass 2)
  int rgroups;  // row groups per slab (partials per slab)
  int npart;    // nslab * rgroups
  int64_t rows_per_slab;
  bool bf16;    // bf16 operand contract (FGMM_FLAG_BF16)
  bool lj;      // pass 1 stores the log-joint; pass 2 reads it (FGMM_FLAG_STORE_LOGJOINT)
  bool autolj;  // the default plan with a stored-log-joint branch that a row-sample probe
                // selects on the device (FGMM_FLAG_STORE_LOGJOINT_AUTO, D <= 128)
  int nprobe;   // sampled 32-row tiles of that probe
  int lj_nh;    // column parts per component block in that pass 2 (1 or 2)
  bool need;    // default plan: pass 1 leaves need masks, pass 2 gathers the needed rows
  bool ctile;   // default plan above D = 128: component-tiled pass 1, dimension-range pass 2
  bool rexact;  // need masks from the block maxima kept in LDS (else the running-max bound)
  int ndr;      // dimension ranges of the component-tiled pass 2 (and of the wide bf16 pass 2)
  bool bfw;     // bf16 contract above D = 256: stored log-joint, iso_bf16_*_wide
  bool bfneed;  // bf16 contract up to D = 128: need masks from pass 1, iso_bf16_gather in pass 2
                // (or iso_bf16_accum where most pairs are needed)
  size_t off_musw, off_mu3, off_kcblk, off_kclin, off_kcgat, off_rowstat, off_part_mu, off_part_nk,
      off_part_sig, off_lj, off_ljmax, off_ljmask, off_ljcount, off_xsplit, off_zpair, off_probe, total;
};

// Pass 1 with need masks keeps a bf16 bound of each row's block maximum in LDS,
// 2 bytes per (row, block) for its 4 waves, while the workgroup still fits twice in
// a compute unit's LDS; for more blocks the masks come from the running-max bound.
__host__ __device__ constexpr size_t lse_lds_base(int DP) {
  return (size_t)2 * (DP / 16) * 4 * 64 * 16 + (size_t)2 * 32 * 16;
}
// Pass 1 with the rows' split operands resident in registers (iso_lse) runs up to
// D = 128 at two waves per SIMD, and at D = 192 and 256 (default plan) at one, with
// four accumulation chains as the component-tiled pass 1 forms them.
__host__ __device__ constexpr bool lse_in_regs(int DP) { return DP <= 128 || DP == 192 || DP == 256; }
__host__ __device__ constexpr int lse_waves_per_simd(int DP) { return DP <= 128 ? 2 : 1; }
// The pipelined pass 1 up to D = 128 is one 8-wave workgroup per compute unit
// (two waves per SIMD) with a third buffer of block constants.
// The pipelined pass 1 of the stored plan also passes each block's log-joint tile
// through LDS (one 32 x 36-float tile per wave), so that its stores are whole lines.
constexpr size_t kPipeStoreLds = (size_t)8 * 32 * 36 * sizeof(float);
__host__ __device__ constexpr int need_exact_cap(int DP) {
  return DP <= 128 ? (int)((kMaxLds - lse_lds_base(DP) - 32 * 16 - 16) / (8 * 32 * 2))
                   : (int)((kMaxLds / (lse_waves_per_simd(DP) == 2 ? 2 : 1) - lse_lds_base(DP)) / (kWaves * 32 * 2));
}

// Pass 2 reads the stored log-joint when it is requested, D is 33 to 256 (below,
// the recomputed contraction costs less than the extra traffic; above, only the
// default plan has kernels), there are at least 4 component blocks, and the tiles
// fit under kMaxLjBytes.
__host__ inline bool use_stored_lj(int64_t N, int DP, int KB, bool allow) {
  return allow && DP >= 64 && DP <= 256 && KB >= 4 &&
         (size_t)round_up(cdiv(N, 32), 4) * (size_t)KB * kLjTile * sizeof(float) <= kMaxLjBytes;
}

// bf16 pass 2: 4 component blocks per workgroup, or 2 / 1 for K <= 64 / 32 where
// the taller X tiles fit in LDS (row-major and transposed bf16, double-buffered).
__host__ __device__ constexpr size_t bf16_accum_lds_bytes(int DP, int CB);
__host__ __device__ constexpr size_t bf16_lse_lds_base(int DP) {
  return (size_t)2 * (DP / 16) * 64 * 16 + (size_t)2 * 32 * 16;   // mu blocks (bf16x8) and constants (f32x4)
}
constexpr int kLjtWavesPlan = 4;   // component blocks per stored pass-2 workgroup up to D = 128 (iso_accum_ljt)
__host__ __device__ constexpr int gather_rs(int DP) { return DP + 16; }   // bf16 row stride of the X tiles
// The stored plan's bf16 X tiles (hi, lo; 32 rows at that stride) up to D = 128.
__host__ __device__ constexpr size_t ljt_xsplit_bytes(int DP) { return (size_t)2 * 32 * gather_rs(DP) * 2; }
// Above D = 256 the bf16 contract stores the log-joint (defined with its kernels).
constexpr int kBwCB = 8;     // component blocks per wide bf16 pass-2 workgroup (one per wave)
constexpr int kBwDR = 256;   // dimensions per wide bf16 pass-2 workgroup
__host__ __device__ constexpr bool iso_bf16_wide(int DP) { return DP > 256; }
__host__ inline size_t bw_lj_bytes(int64_t N, int KP) {
  return (size_t)round_up(cdiv(N, 32), 4) * (size_t)KP * 32 * sizeof(float);
}
__host__ __device__ constexpr int bf16_halves(int DP);
__host__ inline int bf16_blocks_per_group(int DP, int KB);

IsoPlan make_plan(int64_t N, int64_t K, int64_t D, bool allow_lj = false, bool bf16 = false,
                  bool auto_lj = false) {
  IsoPlan p{};
  p.N = N; p.K = K; p.D = D;
  p.DP = iso_padded_dim(D);
  p.KB = (int)cdiv(K, 32);
  p.KP = p.KB * 32;
  p.bf16 = bf16;
  p.lj = !bf16 && use_stored_lj(N, p.DP, p.KB, allow_lj);
  p.need = !bf16 && !p.lj;
  p.autolj = p.need && auto_lj && p.DP <= 128 && N > 0 && p.KB > 0 && p.KB <= kProbeMaxKB &&
             (size_t)round_up(cdiv(N, 32), 8) * (size_t)p.KB * kLjTile * sizeof(float) <= kMaxLjBytes;
  p.nprobe = p.autolj ? (int)std::min<int64_t>(kProbeTiles, cdiv(N, 32)) : 0;
  p.ctile = p.need && p.DP > 128;
  p.rexact = (p.need || (p.lj && p.DP <= 128)) &&
             p.KB <= ((p.ctile && !lse_in_regs(p.DP)) ? ctile_need_exact_cap(ctile_blocks(p.DP))
                      : (p.lj || p.autolj) ? need_exact_cap(p.DP) - (int)(kPipeStoreLds / (8 * 32 * 2))
                                           : need_exact_cap(p.DP));
  p.ndr = p.ctile ? (int)cdiv(p.DP, kDrange) : 1;
  p.bfw = bf16 && iso_bf16_wide(p.DP);
  if (p.bfw) {
    p.cpg = kBwCB;
    p.rgroups = 1;
    p.ndr = (int)cdiv(p.DP, kBwDR);
  } else if (bf16) {
    p.cpg = bf16_blocks_per_group(p.DP, p.KB);
    p.rgroups = kAccWaves / (p.cpg * bf16_halves(p.DP));
  } else if (p.lj && p.DP <= 128) {
    p.cpg = kLjtWavesPlan;   // iso_accum_ljt: one wave per block, 4 blocks per workgroup
    p.lj_nh = 1;
    p.rgroups = 1;
  } else if (p.lj) {
    // 8 component blocks per workgroup, or 4 for K <= 224 and for D > 192; with 4
    // blocks above D = 128 two waves share a block (one half of the columns each):
    // one wave's accumulators for all of D would not fit with the other state.
    p.cpg = (p.KB >= 8 && p.DP <= 192) ? 8 : 4;
    p.lj_nh = (p.DP > 128 && p.cpg == 4) ? 2 : 1;
    p.rgroups = kAccWaves / (p.cpg * p.lj_nh);
  } else {
    p.cpg = 1;        // one wave (D <= 128) or workgroup per (row slab, component block)
    p.rgroups = 1;
  }
  p.ncg = (int)cdiv(p.KB, p.cpg);
  const int64_t tile_rows = 32 * p.rgroups;
  if (p.bfw && N > 0 && p.KB > 0) {
    // About two workgroups per compute unit.
    int64_t want = cdiv((int64_t)2 * current_device_cus(), (int64_t)p.ncg * p.ndr);
    if (want > cdiv(N, 32)) want = cdiv(N, 32);
    p.rows_per_slab = round_up(cdiv(N, want), 32);
    p.nslab = (int)cdiv(N, p.rows_per_slab);
  } else if (p.ctile && N > 0 && p.KB > 0) {
    // One 4-wave workgroup per (slab, block, dimension range) and compute unit (its
    // X tile takes most of the LDS): about two rounds of workgroups.
    int64_t want = cdiv((int64_t)2 * current_device_cus(), (int64_t)p.KB * p.ndr);
    const int64_t max_slabs = cdiv(N, 32);
    if (want > max_slabs) want = max_slabs;
    p.rows_per_slab = cap_slab_rows(round_up(cdiv(N, want), 32), sizeof(double2));
    p.nslab = (int)cdiv(N, p.rows_per_slab);
  } else if (p.need && N > 0 && p.KB > 0) {
    // The gathering pass 2: eight waves per compute unit, two rounds at one wave per
    // SIMD (one round where two fit).
    const int64_t want = gather_slab_count(cdiv((int64_t)8 * current_device_cus(), p.KB), cdiv(N, 32), kGatherWaves);
    p.rows_per_slab = cap_slab_rows(round_up(cdiv(N, want), 32), sizeof(double2));
    p.nslab = (int)cdiv(N, p.rows_per_slab);
  } else if (N > 0 && p.ncg > 0) {
    // One 8-wave workgroup per compute unit; the stored pass 2 up to D = 128 runs two
    // 4-wave workgroups on each.
    int64_t want = (int64_t)current_device_cus() * (p.lj && p.DP <= 128 ? 8 / kLjtWavesPlan : 1) / p.ncg;
    if (want >= 8) want = (want / 8) * 8;  // keeps a slab's workgroups on one XCD
    if (want < 1) want = 1;
    const int64_t max_slabs = cdiv(N, tile_rows);
    if (want > max_slabs) want = max_slabs;
    p.rows_per_slab = round_up(cdiv(N, want), tile_rows);
    if (p.lj && p.DP <= 128) p.rows_per_slab = cap_slab_rows(p.rows_per_slab, sizeof(double2));
    p.nslab = (int)cdiv(N, p.rows_per_slab);
  } else {
    p.rows_per_slab = tile_rows;
    p.nslab = 0;
  }
  p.npart = p.nslab * p.rgroups;
  // The bf16 contract's need masks: each row's block maxima (bf16, 2 bytes per row and
  // block for the 4 waves of a pass-1 workgroup) must fit in LDS beside the stages.
  p.bfneed = bf16 && !p.bfw && p.DP <= 128 && p.KB > 0 &&
             bf16_lse_lds_base(p.DP) + (size_t)kWaves * 32 * p.KB * 2 <= kMaxLds;
  size_t off = 0;
  // The bf16 contract's operands (the fp32 plans read only the split operands below).
  p.off_musw = off;    off = align256(off + (bf16 ? (size_t)p.KP * p.DP * sizeof(float) : 0));
  p.off_mu3 = off;     off = align256(off + (size_t)p.KP * p.DP * 4 * 2);   // bf16 splits of mu
  p.off_kcblk = off;   off = align256(off + (size_t)p.KB * 32 * 2 * sizeof(double));
  p.off_kclin = off;   off = align256(off + (size_t)p.KP * 4 * sizeof(double));
  p.off_kcgat = off;   off = align256(off + (size_t)p.KP * 4 * sizeof(double));
  p.off_rowstat = off; off = align256(off + (size_t)(N > 0 ? N : 0) * 2 * sizeof(double));
  p.off_part_mu = off; off = align256(off + (size_t)p.npart * p.KP * p.DP * sizeof(float));
  p.off_part_nk = off; off = align256(off + (size_t)p.npart * p.KP * sizeof(float));
  p.off_part_sig = off; off = align256(off + (size_t)p.npart * p.KP * sizeof(float));
  // One log-joint tile per pass-1 wave (the grid's 32-row tiles, rounded up to 4),
  // with its per-row block maxima and need mask; the default plan keeps the masks only.
  // (The default plan's pass 1 up to D = 128 runs 8 tiles per workgroup.)
  const bool pipe1 = (p.need || p.lj) && p.DP <= 128;   // pass 1 is iso_lse_pipe (8 tiles per workgroup)
  const size_t ntile = (p.lj || p.need || p.bfneed) ? (size_t)round_up(cdiv(N, 32), pipe1 ? 8 : 4) * p.KB : 0;
  p.off_lj = off;
  off = align256(off + (p.bfw ? bw_lj_bytes(N, p.KP) : (p.lj || p.autolj) ? ntile * kLjTile * sizeof(float) : 0));
  p.off_ljmax = off;  off = align256(off + (p.lj && !pipe1 ? ntile * 32 * sizeof(float) : 0));
  p.off_ljmask = off; off = align256(off + ntile * sizeof(unsigned));
  p.off_ljcount = off; off = align256(off + ((p.lj || p.need || p.bfneed) ? 64 * sizeof(unsigned) : 0));
  // The stored plan up to D = 128: each pass-1 tile's bf16 X parts and logZ2 pairs.
  const size_t ptiles = ((p.lj || p.autolj) && pipe1) ? (size_t)round_up(cdiv(N, 32), 8) : 0;
  p.off_xsplit = off; off = align256(off + ptiles * ljt_xsplit_bytes(p.DP));
  p.off_zpair = off;  off = align256(off + ptiles * 32 * sizeof(float2));
  // The probe: sampled rows' block maxima, its counters and the selector word.
  p.off_probe = off;  off = align256(off + (p.autolj ? probe_bytes() : 0));
  p.total = off;
  return p;
}

// ---------------------------------------------------------------------------
// Prologue: one 64-thread block per 32-component block.
// ---------------------------------------------------------------------------
__global__ __launch_bounds__(64) void iso_prep(const float* __restrict__ mu, int64_t ldmu, int64_t K,
                                               int D, int DP, const float* __restrict__ lss,
                                               const float* __restrict__ lpi, double2* __restrict__ kc_blk, double4* __restrict__ kc_lin,
                                               double4* __restrict__ kc_gat, bf16x8* __restrict__ mu3,
                                               unsigned* __restrict__ ljcount) {
  __shared__ double sC[32], sB[32];
  const int kb = blockIdx.x;
  const int lane = threadIdx.x, c = lane & 31, g = lane >> 5;
  // Pass 1 counts the needed row pairs of the stored log-joint into these.
  if (ljcount && kb == 0) ljcount[lane] = 0u;
  const int64_t comp = (int64_t)kb * 32 + c;
  const bool valid = comp < K;
  const int NQ = DP / 16;
  if (g == 0) {
    double C = -INFINITY, b = 0.0, musq = 0.0, osum = 0.0;
    if (valid) {
      // ||mu||^2 as the sum of the chunks' squared norms, and the centring offsets
      // of the bf16x6 pass 1, o_q = fp32(||mu chunk q||^2).  Each chunk's 16 loads
      // are unrolled so they are in flight together (this kernel runs K / 32 blocks
      // and is latency bound).
      // Loads from clamped addresses with the value selected after, so no load waits
      // behind a branch.
#pragma unroll 2
      for (int q = 0; q < NQ; ++q) {
        double o = 0.0;
#pragma unroll
        for (int e = 0; e < 16; ++e) {
          const int d = 16 * q + e;
          const float f = mu[comp * ldmu + (d < D ? d : D - 1)];
          const double v = d < D ? (double)f : 0.0;
          o = fma(v, v, o);
        }
        musq += o;
        osum += (double)(float)o;
      }
      const double l = (double)lss[comp];
      const double lp = (double)lpi[comp];
      b = 0.5 * exp(-l) * kLog2e;
      C = (lp - 0.5 * (double)D * (kLog2Pi + l)) * kLog2e - b * musq;
    }
    // The split-bf16 passes contract the centred cross term x.mu - sum_q o_q, so
    // their constant carries + 2 b sum_q o_q.
    sC[c] = valid ? C + 2.0 * b * osum : C;
    sB[c] = b;
    kc_lin[comp] = make_double4(C, b, musq, 0.0);
    // The gathering passes 2 take the centred constant and, for
    // ||x - mu||^2 = ||x||^2 - 2 (x.mu - sum_q o_q) + (||mu||^2 - 2 sum_q o_q), the last term.
    kc_gat[comp] = make_double4(sC[c], b, musq - 2.0 * osum, 0.0);
  }
  // The same chunks as three-way bf16 splits for the bf16x6 pass 1,
  // mu3[kb][q][s][lane] = split s of mu[comp][16q + 8g .. 16q + 8g + 7] (s < 3), and
  // slot 3 = the splits of -o_q in k slots 0..2 (lane-half 0, elements 0..2).
  for (int q = 0; q < NQ; ++q) {
    f32x4 lo = zero4(), hi = zero4();
    const int d0 = 16 * q + 8 * g;
    if (valid) {
#pragma unroll
      for (int e = 0; e < 4; ++e) {
        const float a = mu[comp * ldmu + (d0 + e < D ? d0 + e : D - 1)];
        const float b = mu[comp * ldmu + (d0 + 4 + e < D ? d0 + 4 + e : D - 1)];
        lo[e] = d0 + e < D ? a : 0.0f;
        hi[e] = d0 + 4 + e < D ? b : 0.0f;
      }
    }
    bf16x8 sp[3];
    split3_bf16(lo, hi, sp);
#pragma unroll
    for (int t = 0; t < 3; ++t) mu3[(((int64_t)kb * NQ + q) * 4 + t) * 64 + lane] = sp[t];
    f32x4 olo = zero4();
    if (valid && g == 0) {
      double o = 0.0;
#pragma unroll
      for (int e = 0; e < 16; ++e) {
        const int d = 16 * q + e;
        const float f = mu[comp * ldmu + (d < D ? d : D - 1)];
        const double v = d < D ? (double)f : 0.0;
        o = fma(v, v, o);
      }
      olo.x = -(float)o;
    }
    bf16x8 so[3];
    split3_bf16(olo, zero4(), so);
    bf16x8 ov;
#pragma unroll
    for (int e = 0; e < 8; ++e) ov[e] = (__bf16)0.0f;
    ov[0] = so[0][0];
    ov[1] = so[1][0];
    ov[2] = so[2][0];
    mu3[(((int64_t)kb * NQ + q) * 4 + 3) * 64 + lane] = ov;
  }
  __syncthreads();
  // Constants in accumulator-register order: entry (g, i) is component acc_row(i, g).
  {
    const int i = lane & 15, gg = (lane >> 4) & 1;
    if (lane < 32) {
      const int cc = acc_row(i, gg);
      kc_blk[((int64_t)kb * 2 + gg) * 16 + i] = make_double2(sC[cc], sB[cc]);
    }
  }
}

// ---------------------------------------------------------------------------
// Pass 1: logZ by online log-sum-exp over component blocks.
// Each wave keeps 32 rows of X in registers as three-way bf16 splits (the
// matrix-core B operand of the centred bf16x6 contraction, x6c_tile).  The
// 32-component blocks of mu (bf16 splits and centring offsets) and their
// constants stream through LDS, double buffered: the global loads of block kb+1
// are in flight while block kb is contracted, and land in the other buffer before
// the block's barrier.
// ---------------------------------------------------------------------------
template <int DP>
constexpr size_t lse_lds_bytes() {
  static_assert(lse_lds_base(DP) == (size_t)2 * (DP / 16) * 4 * 64 * sizeof(bf16x8) + (size_t)2 * 32 * sizeof(double2),
                "pass-1 LDS");
  return lse_lds_base(DP);
}

// Accumulation chains of the split-bf16 contraction (x6c_tile, x6c_tile_rows): pass 1
// and the recomputing pass 2 use the same number, so they form the same sums.
constexpr int kIsoChains = 2;

// What pass 1 leaves for pass 2 besides logZ2 and ||x||^2.
constexpr int kLjmStore = 1;   // the stored log-joint, its block maxima and need masks
constexpr int kLjmNeed = 2;    // need masks only (the default plan)

template <int DP, int LJM>
__global__ __attribute__((amdgpu_flat_work_group_size(kThreads, kThreads),
                          amdgpu_waves_per_eu(lse_waves_per_simd(DP), lse_waves_per_simd(DP))))
void iso_lse(const float* __restrict__ X, int64_t ldx, int64_t N, int D,
             const bf16x8* __restrict__ mu3, const double2* __restrict__ kc_blk, int KB,
             float* __restrict__ logZ, double2* __restrict__ rowstat, float* __restrict__ lj,
             float* __restrict__ ljmax, unsigned* __restrict__ ljmask, unsigned* __restrict__ ljcount,
             int dense, int rexact) {
  constexpr int NQ = DP / 16;
  constexpr int BLK = NQ * 4 * 64;        // bf16x8 per 32-component block
  constexpr int LPT = (BLK + kThreads - 1) / kThreads;
  constexpr bool LJ = LJM == kLjmStore;

  extern __shared__ __align__(16) unsigned char lds_raw[];
  bf16x8* mu_l = reinterpret_cast<bf16x8*>(lds_raw);                                 // [2][BLK]
  double2* kc_l = reinterpret_cast<double2*>(lds_raw + 2 * BLK * sizeof(bf16x8));   // [2][32]
  // Need masks: the rows' block-maximum bounds, [wave][block][row] (rexact only).
  unsigned short* rmax_l = reinterpret_cast<unsigned short*>(lds_raw + lse_lds_bytes<DP>());

  const int tid = threadIdx.x, lane = tid & 63;
  const int wave = __builtin_amdgcn_readfirstlane(tid >> 6);   // uniform: tile bases in scalars
  const int c = lane & 31, g = lane >> 5;
  const int64_t tile = (int64_t)blockIdx.x * kWaves + wave;   // 32-row tile
  const int64_t row = tile * 32 + c;
  const bool valid = row < N;

  bf16x8 st[LPT];
  double2 kst = make_double2(0.0, 0.0);
  // Buffer loads from a resource per block: the lane's offset is loop-invariant and
  // the per-load part is a scalar, so the fetch costs no vector address arithmetic.
  auto fetch = [&](int kb) {
    const buf_rsrc r = make_rsrc(mu3 + (int64_t)kb * BLK, (uint32_t)(BLK * sizeof(bf16x8)));
#pragma unroll
    for (int q = 0; q < LPT; ++q)
      st[q] = __builtin_bit_cast(bf16x8, __builtin_amdgcn_raw_buffer_load_b128(
                                             r, tid * (int)sizeof(bf16x8), q * kThreads * (int)sizeof(bf16x8), 0));
    if (tid < 32) kst = kc_blk[(int64_t)kb * 32 + tid];
  };
  auto commit = [&](int buf) {
#pragma unroll
    for (int q = 0; q < LPT; ++q)
      if (BLK % kThreads == 0 || q * kThreads + tid < BLK) mu_l[buf * BLK + q * kThreads + tid] = st[q];
    if (tid < 32) kc_l[buf * 32 + tid] = kst;
  };
  fetch(0);

  // This lane's row, dimensions 16q + 8g .. +7, split three ways; ||x||^2 in fp64.
  bf16x8 xb[NQ][3];
  double xsq = 0.0;
#pragma unroll
  for (int q = 0; q < NQ; ++q) {
    const int d0 = 16 * q + 8 * g;
    const f32x4 lo = load_row4(X, ldx, row, d0, D, valid), hi = load_row4(X, ldx, row, d0 + 4, D, valid);
#pragma unroll
    for (int e = 0; e < 4; ++e) {
      xsq = fma((double)lo[e], (double)lo[e], xsq);
      xsq = fma((double)hi[e], (double)hi[e], xsq);
    }
    split3_bf16(lo, hi, xb[q]);
  }
  xsq += __shfl_xor(xsq, 32);
  const bf16x8 ones = x6c_ones(lane);
  commit(0);
  lds_barrier();

  double mx = -INFINITY;
  float sm = 0.0f;
  float run_max = -INFINITY;   // running max of the row's stored log-joint / block maxima
  unsigned pairs = 0;          // needed rows over the blocks (need masks from the running max)

  for (int kb = 0; kb < KB; ++kb) {
    const int buf = kb & 1;
    const bool more = kb + 1 < KB;
    if (more) fetch(kb + 1);
    const bf16x8* mp = mu_l + buf * BLK + lane;
    // Centred S^T[comp][row] = mu . x - sum_q o_q, lane = row, register i = component
    // acc_row(i, g); the block's constants carry + 2 b sum_q o_q.
    const f32x16 xm = x6c_tile<NQ, (DP <= 128 ? kIsoChains : 4)>([&](int q, int t) { return mp[(q * 4 + t) * 64]; },
                                                                   xb, ones);
    const double2* kp = kc_l + buf * 32 + g * 16;
    double ll[16];
    double bm = -INFINITY;
#pragma unroll
    for (int i = 0; i < 16; ++i) {
      const double2 cb = kp[i];
      ll[i] = fma(-cb.y, fma(-2.0, (double)xm[i], xsq), cb.x);
      bm = fmax(bm, ll[i]);
    }
    // Keep the max here: sunk past the conditional commit below, its operands
    // would cross a block boundary and each cost a canonicalising max.
    asm volatile("" : "+v"(bm));
    const double mn = fmax(mx, bm);
    const double ms = (mn == -INFINITY) ? 0.0 : mn;
    float acc = sm * fast_exp2((float)(mx - ms));
#pragma unroll
    for (int i = 0; i < 16; ++i) acc += fast_exp2((float)(ll[i] - ms));
    sm = acc;
    mx = mn;
    // Tiles are allocated for the whole grid, rows past N included.
    if constexpr (LJ)
      lj_put_rows(lj + (tile * KB + kb) * kLjTile, ljmax + (tile * KB + kb) * 32, c, g, ll, bm, acc,
                  run_max, dense != 0);
    if constexpr (LJM == kLjmNeed) {
      const float R = lj_row_max(bm);   // the row's block maximum, in both half-waves
      if (rexact) {
        if (g == 0) rmax_l[(wave * KB + kb) * 32 + c] = bf16_bits_up(R);
      } else {
        // logZ2 >= the row's final maximum >= run_max - 1 ulp, so a block whose maximum is
        // kLjSkipGap below the running max cannot reach the test of need_put_masks.
        run_max = fmaxf(run_max, R);
        const bool nb = valid && (dense != 0 || !(R - run_max < -kLjSkipGap));
        const unsigned bits = (unsigned)__builtin_amdgcn_ballot_w64(nb);
        if (lane == 0) ljmask[tile * KB + kb] = bits;
        pairs += __builtin_popcount(bits);
      }
    }
    if (more) commit(buf ^ 1);
    lds_barrier();
  }

  // Merge the two half-waves that hold the same row.
  const double mo = __shfl_xor(mx, 32);
  const float so = __shfl_xor(sm, 32);
  const double mn = fmax(mx, mo);
  const double ms = (mn == -INFINITY) ? 0.0 : mn;
  const float tot = sm * fast_exp2((float)(mx - ms)) + so * fast_exp2((float)(mo - ms));
  const double lz2 = mn + (double)log2f(tot);
  if (valid && g == 0) {
    rowstat[row] = make_double2(xsq, lz2);
    if (logZ) logZ[row] = (float)(lz2 * kLn2);
  }
  if constexpr (LJ) {
    if (g == 0) lj_put_masks(ljmax + tile * KB * 32, ljmask + tile * KB, ljcount + (tile & 63), KB, c, lz2,
                   valid, dense != 0);
  }
  if constexpr (LJM == kLjmNeed) {
    if (rexact) {
      const unsigned short* rm = rmax_l + wave * KB * 32 + c;
      if (g == 0)
        need_put_masks([&](int kb) { return bf16_bits_to_float(rm[kb * 32]); }, ljmask + tile * KB,
                       ljcount + (tile & 63), KB, c, lz2, valid, dense != 0);
    } else {
      // A row whose logZ2 is NaN (a NaN log-joint somewhere) gets its bit in every
      // block, as the exact test gives it.
      const unsigned nanbits = (unsigned)__builtin_amdgcn_ballot_w64(valid && g == 0 && lz2 != lz2);
      if (lane == 0) {
        if (nanbits != 0)
          for (int kb = 0; kb < KB; ++kb) ljmask[tile * KB + kb] |= nanbits;
        if (pairs != 0) atomicAdd(ljcount + (tile & 63), pairs);
      }
    }
  }
}

// ---------------------------------------------------------------------------
// Pass 1 of the default plan up to D = 128, software-pipelined in ping-pong.  The
// arithmetic is iso_lse's (same contraction, chains, fp64 log-joint, online
// log-sum-exp and need bounds), so logZ2 and the need bits are the same bits; only
// the schedule differs.
//
// On gfx950 a matrix step leaves the SIMD's issue free for part of its 32 cycles,
// and another wave's VALU instructions run there.  iso_lse's two waves per SIMD
// fall into step (both contracting a block, then both in its epilogue), so little
// of that overlap happens.  Here one workgroup of 8 waves holds 256 rows, two
// waves per SIMD, and each iteration does the contraction of block kb and the
// epilogue (log-joint, max, exp2 sum, need bound) of block kb - 1 in opposite
// orders on the two waves of a SIMD: one contracts first, the other runs the
// epilogue first.  The workgroup barrier at the end of each block keeps them in
// opposite phase, so one wave's VALU work fills the other's matrix steps.  Roles
// come from the hardware wave id's SIMD field, one of each per SIMD (the first
// wave of a SIMD to arrive takes the contract-first role), so the pairing does not
// depend on how the dispatcher places waves.  The mu blocks reach LDS by direct
// buffer-to-LDS loads (no staging registers), double buffered; the constants are
// triple buffered, since block kb - 1's are read while block kb + 1's arrive.
// The eight 32-row tiles share one staging of each mu block.
//
// Workgroups below `full` take 8 tiles each (whole rounds of one workgroup per compute
// unit); the rest take `small` tiles each, so that the tiles left after the last whole
// round spread over every compute unit instead of a few workgroups of 8.  A wave of
// such a group without a tile (wave >= small, or past the last tile) is idle: it issues
// its share of the block loads and meets every barrier, and computes and writes
// nothing.
// ---------------------------------------------------------------------------
constexpr int kPipeWaves = 8;
constexpr int kPipeThreads = 64 * kPipeWaves;

// iso_lse_pipe's grid: whole rounds of 8-tile workgroups (one per compute unit),
// then the tiles left in groups of `small`, one group per compute unit.
struct PipeGrid {
  int64_t grid, full;
  int small;
};
__host__ inline PipeGrid pipe_grid(int64_t N) {
  const int64_t T = cdiv(N, 32), G = cdiv(T, kPipeWaves), cus = current_device_cus();
  PipeGrid pg{G, G, kPipeWaves};
  const int64_t F = T / (kPipeWaves * cus);
  const int64_t R = T - F * kPipeWaves * cus;
  if (F > 0 && R > 0) {
    pg.small = (int)cdiv(R, cus);
    pg.full = F * cus;
    pg.grid = pg.full + cdiv(R, (int64_t)pg.small);
  }
  return pg;
}

template <int DP>
constexpr size_t lse_pipe_lds_bytes() {
  return (size_t)2 * (DP / 16) * 4 * 64 * sizeof(bf16x8) + (size_t)3 * 32 * sizeof(double2) + 16;
}

template <int DP, int REXACT>
__global__ __attribute__((amdgpu_flat_work_group_size(kPipeThreads, kPipeThreads), amdgpu_waves_per_eu(2, 2)))
void iso_lse_pipe(const float* __restrict__ X, int64_t ldx, int64_t N, int D,
                  const bf16x8* __restrict__ mu3, const double2* __restrict__ kc_blk, int KB,
                  float* __restrict__ logZ, double2* __restrict__ rowstat, unsigned* __restrict__ ljmask,
                  unsigned* __restrict__ ljcount, int dense, float* __restrict__ lj,
                  ProbeSel probe, __bf16* __restrict__ xsplit, float2* __restrict__ zpair, int64_t full,
                  int small) {
  static_assert(DP <= 128, "pipelined pass 1 keeps all of a row's splits in registers");
  constexpr int NQ = DP / 16;
  constexpr int BLK = NQ * 4 * 64;        // bf16x8 per 32-component block
  constexpr int LPT = (BLK + kPipeThreads - 1) / kPipeThreads;

  extern __shared__ __align__(16) unsigned char lds_raw[];
  bf16x8* mu_l = reinterpret_cast<bf16x8*>(lds_raw);                                 // [2][BLK]
  double2* kc_l = reinterpret_cast<double2*>(lds_raw + 2 * BLK * sizeof(bf16x8));   // [3][32]
  unsigned* simd_l = reinterpret_cast<unsigned*>(kc_l + 3 * 32);                     // [4]
  unsigned short* rmax_l = reinterpret_cast<unsigned short*>(lds_raw + lse_pipe_lds_bytes<DP>());
  // Stored plan: the wave's log-joint tile on its way to memory (after the bounds).
  float* tr_l = reinterpret_cast<float*>(lds_raw + lse_pipe_lds_bytes<DP>() +
                                         (REXACT ? (size_t)kPipeWaves * 32 * KB * 2 : 0));

  const int tid = threadIdx.x, lane = tid & 63;
  const int wave = __builtin_amdgcn_readfirstlane(tid >> 6);
  const int c = lane & 31, g = lane >> 5;
  const bool tail = (int64_t)blockIdx.x >= full;
  const int64_t tile = tail ? full * kPipeWaves + ((int64_t)blockIdx.x - full) * small + wave
                            : (int64_t)blockIdx.x * kPipeWaves + wave;
  const bool idle = tail && (wave >= small || tile * 32 >= N);
  const int64_t row = tile * 32 + c;
  const bool valid = !idle && row < N;
  // Whether this call stores the log-joint: never without lj, always without a
  // probe, else as the probe's counts (written before this kernel) say.
  const bool store = lj != nullptr && (probe.count == nullptr || probe_selects(probe));

  // Block kb's operands into mu buffer kb & 1, its constants into kc buffer kb % 3.
  // A lane whose piece lies past the block (BLK not a multiple of the workgroup's
  // 512 lanes) is switched off rather than given an out-of-range offset, which
  // would write zeros into LDS.
  auto fetch = [&](int kb) {
    const DmaSrc r = dma_src(mu3 + (int64_t)kb * BLK, (uint32_t)(BLK * sizeof(bf16x8)));
    bf16x8* dst = mu_l + (kb & 1) * BLK + wave * 64;
#pragma unroll
    for (int q = 0; q < LPT; ++q) {
      if (BLK % kPipeThreads == 0 || q * kPipeThreads + wave * 64 < BLK)
        lds_dma16(r, dst + q * kPipeThreads, tid * (int)sizeof(bf16x8), q * kPipeThreads * (int)sizeof(bf16x8));
    }
    if (wave == 0) {
      if (lane < 32) {
        const DmaSrc rk = dma_src(kc_blk + (int64_t)kb * 32, (uint32_t)(32 * sizeof(double2)));
        lds_dma16(rk, kc_l + (kb % 3) * 32, lane * (int)sizeof(double2), 0);
      }
    }
  };
  if (tid < 4) simd_l[tid] = 0u;
  fetch(0);

  bf16x8 xb[NQ][3];
  double xsq = 0.0;
#pragma unroll
  for (int q = 0; q < NQ; ++q) {
    const int d0 = 16 * q + 8 * g;
    const f32x4 lo = load_row4(X, ldx, row, d0, D, valid), hi = load_row4(X, ldx, row, d0 + 4, D, valid);
#pragma unroll
    for (int e = 0; e < 4; ++e) {
      xsq = fma((double)lo[e], (double)lo[e], xsq);
      xsq = fma((double)hi[e], (double)hi[e], xsq);
    }
    split3_bf16(lo, hi, xb[q]);
  }
  xsq += __shfl_xor(xsq, 32);
  const bf16x8 ones = x6c_ones(lane);
  lds_barrier();   // simd_l cleared
  // HW_ID bits 5:4 are the wave's SIMD.  The first wave of a SIMD to arrive
  // contracts first; the second runs the epilogue first.
  const int simd = (__builtin_amdgcn_s_getreg((4) | (0 << 6) | ((32 - 1) << 11)) >> 4) & 3;
  unsigned order = 0;
  if (lane == 0) order = atomicAdd(simd_l + simd, 1u);
  const bool epi_first = __builtin_amdgcn_readfirstlane(order) != 0;
  dma_barrier();

  auto contract = [&](int kb) {
    const bf16x8* mp = mu_l + (kb & 1) * BLK + lane;
    return x6c_tile<NQ, kIsoChains>([&](int q, int t) { return mp[(q * 4 + t) * 64]; }, xb, ones);
  };

  double mx = -INFINITY;
  float sm = 0.0f;
  float run_max = -INFINITY;
  unsigned pairs = 0;
  // Log-joint, block max and exp2 sum of block kb (its contraction in xm), as iso_lse
  // forms them; returns the row's block maximum over both half-waves.  When storing,
  // the lane's 16 values go to the block's tile (row-major, one 128-byte line per
  // row).
  auto epilogue = [&](int kb, const f32x16& xm) {
    const double2* kp = kc_l + (kb % 3) * 32 + g * 16;
    // All 16 constant reads in flight before the first is used.
    double2 cb[16];
#pragma unroll
    for (int i = 0; i < 16; ++i) cb[i] = kp[i];
    __builtin_amdgcn_sched_barrier(0);
    double ll[16];
    double bm = -INFINITY;
#pragma unroll
    for (int i = 0; i < 16; ++i) {
      ll[i] = fma(-cb[i].y, fma(-2.0, (double)xm[i], xsq), cb[i].x);
      bm = fmax(bm, ll[i]);
    }
    const double mn = fmax(mx, bm);
    const double ms = (mn == -INFINITY) ? 0.0 : mn;
    float acc = sm * fast_exp2((float)(mx - ms));
#pragma unroll
    for (int i = 0; i < 16; ++i) acc += fast_exp2((float)(ll[i] - ms));
    sm = acc;
    mx = mn;
    const float R = lj_row_max(bm);
    if (store) {
      // Every row of every block, so that each epilogue issues exactly four store
      // instructions (the block barrier's wait leaves these in flight); a row past N
      // lands in the padding of the last tiles.  The tile is transposed through the
      // wave's LDS tile (row stride 36 floats) so that each store writes 8 whole rows.
      float* tl = tr_l + wave * 32 * 36;
#pragma unroll
      for (int j = 0; j < 4; ++j) {
        const f32x4 v = {(float)ll[4 * j], (float)ll[4 * j + 1], (float)ll[4 * j + 2], (float)ll[4 * j + 3]};
        *reinterpret_cast<f32x4*>(tl + c * 36 + 8 * j + 4 * g) = v;
      }
      float* p = lj + (tile * KB + kb) * kLjTile;
#pragma unroll
      for (int q = 0; q < 4; ++q) {
        const int rr = 8 * q + (lane >> 3), cc = 4 * (lane & 7);
        *reinterpret_cast<f32x4*>(p + rr * 32 + cc) = *reinterpret_cast<const f32x4*>(tl + rr * 36 + cc);
      }
    }
    return R;
  };
  // The need bound of block kb: kept in LDS (REXACT) or tested against the running
  // max.  Both half-waves store the row's bound (the same value); the mask word goes
  // out through a buffer store whose offset is out of range on every lane but 0.
  const buf_rsrc mask_r = make_rsrc(ljmask + tile * KB, (uint32_t)(KB * sizeof(unsigned)));
  const int mask_off = buf_off(lane == 0 ? 0 : kBufOob);
  auto put_need = [&](int kb, float R) {
    if constexpr (REXACT) {
      rmax_l[(wave * KB + kb) * 32 + c] = bf16_bits_up(R);
    } else {
      run_max = fmaxf(run_max, R);
      const bool nb = valid && (dense != 0 || !(R - run_max < -kLjSkipGap));
      const unsigned bits = (unsigned)__builtin_amdgcn_ballot_w64(nb);
      __builtin_amdgcn_raw_buffer_store_b32(bits, mask_r, mask_off, kb * (int)sizeof(unsigned), 0);
      pairs += __builtin_popcount(bits);
    }
  };

  if (idle) {
    // Its share of every block's loads and every barrier (the active waves meet no
    // barrier after the block loop), nothing else.
    if (KB > 1) fetch(1);
    dma_barrier();
    for (int kb = 1; kb < KB; ++kb) {
      if (kb + 1 < KB) fetch(kb + 1);
      dma_barrier();
    }
    return;
  }
  if (KB > 1) fetch(1);
  f32x16 xm = contract(0);
  dma_barrier();
  for (int kb = 1; kb < KB; ++kb) {
    if (kb + 1 < KB) fetch(kb + 1);
    f32x16 xn;
    float R;
    if (epi_first) {
      R = epilogue(kb - 1, xm);
      __builtin_amdgcn_sched_barrier(0);
      xn = contract(kb);
    } else {
      xn = contract(kb);
      __builtin_amdgcn_sched_barrier(0);
      R = epilogue(kb - 1, xm);
    }
    put_need(kb - 1, R);
    xm = xn;
    // Block kb + 1's operands have landed once at most this iteration's stores (the
    // log-joint's four, the mask word's one) are in flight: the stores of a block
    // complete behind the next block's contraction.
    if (store) {
      if constexpr (REXACT) asm volatile("s_waitcnt vmcnt(4) lgkmcnt(0)\n\ts_barrier" ::: "memory");
      else asm volatile("s_waitcnt vmcnt(5) lgkmcnt(0)\n\ts_barrier" ::: "memory");
    } else {
      if constexpr (REXACT) dma_barrier();
      else asm volatile("s_waitcnt vmcnt(1) lgkmcnt(0)\n\ts_barrier" ::: "memory");
    }
  }
  put_need(KB - 1, epilogue(KB - 1, xm));

  // Merge the two half-waves that hold the same row.
  const double mo = __shfl_xor(mx, 32);
  const float so = __shfl_xor(sm, 32);
  const double mn = fmax(mx, mo);
  const double ms = (mn == -INFINITY) ? 0.0 : mn;
  const float tot = sm * fast_exp2((float)(mx - ms)) + so * fast_exp2((float)(mo - ms));
  const double lz2 = mn + (double)log2f(tot);
  if (valid && g == 0) {
    rowstat[row] = make_double2(xsq, lz2);
    if (logZ) logZ[row] = (float)(lz2 * kLn2);
  }
  if (store) {
    // The tile's bf16 (hi, lo) parts of X for the stored plan's pass 2, row-major
    // with its LDS row stride (ljt_xsplit_bytes per tile).  Written last, so that no
    // wait of the block loop covers them.
    __bf16* xp = xsplit + tile * (2 * 32 * gather_rs(DP)) + c * gather_rs(DP) + 8 * g;
#pragma unroll
    for (int q = 0; q < NQ; ++q) {
      *reinterpret_cast<bf16x8*>(xp + 16 * q) = xb[q][0];
      *reinterpret_cast<bf16x8*>(xp + 32 * gather_rs(DP) + 16 * q) = xb[q][1];
    }
    if (g == 0) {
      // logZ2 as the (hi, lo) float pair the stored plan's pass 2 subtracts; +inf
      // for a row past N, whose responsibilities are then exactly 0 there.
      const float zh = valid ? (float)lz2 : INFINITY;
      const float zl = (valid && lz2 > -INFINITY && lz2 < INFINITY) ? (float)(lz2 - (double)zh) : 0.0f;
      zpair[tile * 32 + c] = make_float2(zh, zl);
    }
  }
  if constexpr (REXACT) {
    // Each lane reads back the bounds it wrote itself.
    const unsigned short* rm = rmax_l + wave * KB * 32 + c;
    if (g == 0)
      need_put_masks([&](int kb) { return bf16_bits_to_float(rm[kb * 32]); }, ljmask + tile * KB,
                     ljcount + (tile & 63), KB, c, lz2, valid, dense != 0);
  } else {
    const unsigned nanbits = (unsigned)__builtin_amdgcn_ballot_w64(valid && g == 0 && lz2 != lz2);
    if (lane == 0) {
      if (nanbits != 0)
        for (int kb = 0; kb < KB; ++kb) ljmask[tile * KB + kb] |= nanbits;
      if (pairs != 0) atomicAdd(ljcount + (tile & 63), pairs);
    }
  }
}

// ---------------------------------------------------------------------------
// The probe of FGMM_FLAG_STORE_LOGJOINT_AUTO (up to D = 128): one workgroup per
// sampled 32-row tile; its waves take the component blocks in turn and form each
// row's block maximum R of the log-joint in LDS.  An estimate suffices here, so
// the contraction keeps two of pass 1's seven steps per 16-dimension chunk (the
// centring step and x1 mu1: an error of a fraction of a log2 unit against the
// kLjNeedGap = 160 margin).  Then, per row, the blocks with R >= M - kLjNeedGap (M
// the row's largest R) are counted: an estimate of the pairs pass 1 will mark as
// needed, since logZ2 >= M.  The tile's count is written; no atomics: the kernels
// that need the choice sum the counts themselves (probe_selects).
// ---------------------------------------------------------------------------
constexpr int kProbeWaves = 16;
template <int DP>
__global__ __launch_bounds__(64 * kProbeWaves) void iso_store_probe(const float* __restrict__ X, int64_t ldx,
                                                                    int64_t N, int D,
                                                                    const bf16x8* __restrict__ mu3,
                                                                    const double2* __restrict__ kc_blk, int KB,
                                                                    int ntile, unsigned* __restrict__ count) {
  constexpr int NQ = DP / 16;
  constexpr int BLK = NQ * 4 * 64;
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
  double xsq = 0.0;
#pragma unroll
  for (int q = 0; q < NQ; ++q) {
    const int d0 = 16 * q + 8 * g;
    const f32x4 lo = load_row4(X, ldx, row, d0, D, valid), hi = load_row4(X, ldx, row, d0 + 4, D, valid);
#pragma unroll
    for (int e = 0; e < 4; ++e) {
      xsq = fma((double)lo[e], (double)lo[e], xsq);
      xsq = fma((double)hi[e], (double)hi[e], xsq);
    }
    xh[q] = to_bf16x8(lo, hi);
  }
  xsq += __shfl_xor(xsq, 32);
  const bf16x8 ones = x6c_ones(lane);
  for (int kb = wave; kb < KB; kb += kProbeWaves) {
    const bf16x8* mp = mu3 + (int64_t)kb * BLK + lane;
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
    const double2* kp = kc_blk + (int64_t)kb * 32 + g * 16;
    double bm = -INFINITY;
#pragma unroll
    for (int i = 0; i < 16; ++i) {
      const double2 cb = kp[i];
      const float xm = (acc[0][i] + acc[1][i]) + (acc[2][i] + acc[3][i]);
      bm = fmax(bm, fma(-cb.y, fma(-2.0, (double)xm, xsq), cb.x));
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
// Pass 1 of the default plan above D = 128 (any D).  The split operands of a row
// no longer fit in registers for all of D, so the contraction is tiled over the
// components as well: each wave owns a 32-row tile, and for each component tile of
// CTB blocks (ctile_blocks) it streams its rows' chunks of 16 dimensions
// from global memory (read once per component tile; from L2 or the MALL after the
// first), splits them three ways into bf16 as they arrive and contracts them with
// the tile's mu operands (bf16 splits and centring offsets), which the
// workgroup's four waves share through an LDS double buffer of two-chunk stages.
// Chunk q accumulates into chain q % 4 of each block with x6c_tile's products and
// order; after the last chunk the chains are added as ((c0 + c1) + c2) + c3, and
// the online log-sum-exp and the need bounds proceed as in iso_lse.  CTB blocks x
// four chains take 64 CTB accumulator registers: two waves per SIMD with 2 blocks,
// one with 4.  The stored
// plan (LJM = kLjmStore, D up to 256) runs the same kernel and also writes the
// log-joint rows, their block maxima and the need masks, as iso_lse does.
// ---------------------------------------------------------------------------
template <int LJM, int CTB>
__global__ __attribute__((amdgpu_flat_work_group_size(64 * kCtWaves, 64 * kCtWaves),
                          amdgpu_waves_per_eu(CTB == 2 ? 2 : 1, CTB == 2 ? 2 : 1)))
void iso_lse_ctile(const float* __restrict__ X, int64_t ldx, int64_t N, int D, int NQ,
                   const bf16x8* __restrict__ mu3, const double2* __restrict__ kc_blk, int KB,
                   float* __restrict__ logZ, double2* __restrict__ rowstat, float* __restrict__ lj,
                   float* __restrict__ ljmax, unsigned* __restrict__ ljmask, unsigned* __restrict__ ljcount,
                   int dense, int rexact) {
  constexpr bool LJ = LJM == kLjmStore;
  constexpr int SO = ctile_stage_ops(CTB);   // bf16x8 per two-chunk operand stage
  constexpr int NT = 64 * kCtWaves;
  constexpr int LPT = SO / NT;   // operand loads per thread per stage
  static_assert(SO % NT == 0 && CTB * 32 <= NT, "stage split");

  extern __shared__ __align__(16) unsigned char lds_raw[];
  bf16x8* mu_l = reinterpret_cast<bf16x8*>(lds_raw);                                        // [2][stage]
  double2* kc_l = reinterpret_cast<double2*>(lds_raw + 2 * SO * sizeof(bf16x8));   // [2][blocks*32]
  unsigned short* rmax_l = reinterpret_cast<unsigned short*>(lds_raw + lse_ctile_base(CTB));  // [wave][KB][32]

  const int tid = threadIdx.x, lane = tid & 63;
  const int wave = __builtin_amdgcn_readfirstlane(tid >> 6);
  const int c = lane & 31, g = lane >> 5;
  const int64_t tile = (int64_t)blockIdx.x * kCtWaves + wave;   // 32-row tile
  const int64_t row = tile * 32 + c;
  const bool valid = row < N;
  const int NS = NQ / 2;                        // stages per component tile (even: NQ % 4 == 0)
  const int nstage = (int)cdiv(KB, CTB) * NS;
  const int nq_full = D / 16;                   // chunks that end at or before D

  // Stage s = (component tile s / NS, chunk pair s % NS).  Thread element u covers
  // block u / 2 of the tile and entry (u % 2) * NT + tid of its 512 = (chunk in the
  // pair, split, lane): the same order in LDS, so operand (b, qq, t) of a lane is
  // at b * 512 + (qq * 4 + t) * 64 + lane.  Blocks at or past KB read zero.
  const int64_t blk_ops = (int64_t)NQ * 4 * 64;     // bf16x8 per block
  const int64_t all_ops = (int64_t)KB * blk_ops;
  bf16x8 st[LPT];
  double2 kst = make_double2(-INFINITY, 0.0);
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
      kst = kc < (int64_t)KB * 32 ? kc_blk[kc] : make_double2(-INFINITY, 0.0);
    }
  };
  auto commit = [&](int s, int buf) __attribute__((always_inline)) {
    const int ct = s / NS, sp = s - ct * NS;
#pragma unroll
    for (int u = 0; u < LPT; ++u) mu_l[buf * SO + u * NT + tid] = st[u];
    if (sp == 0 && tid < CTB * 32) kc_l[(ct & 1) * CTB * 32 + tid] = kst;
  };

  // The wave's rows, dimensions 16q + 8g .. + 7 of chunk q (zero past D and N).
  const float* xrow = X + (valid ? row : 0) * ldx + 8 * g;
  auto xload = [&](int q, f32x4& lo, f32x4& hi) __attribute__((always_inline)) {
    if (q < nq_full) {
      lo = *reinterpret_cast<const f32x4*>(xrow + 16 * q);
      hi = *reinterpret_cast<const f32x4*>(xrow + 16 * q + 4);
      if (!valid) { lo = zero4(); hi = zero4(); }
    } else {
      lo = load_row4(X, ldx, row, 16 * q + 8 * g, D, valid);
      hi = load_row4(X, ldx, row, 16 * q + 8 * g + 4, D, valid);
    }
  };
  f32x4 xr[2][2][2];   // [stage parity][chunk in the pair][lo, hi]
  auto xstage = [&](int s, f32x4 (&dst)[2][2]) __attribute__((always_inline)) {
    if (s >= nstage) return;
    const int sp = s % NS;
    xload(2 * sp, dst[0][0], dst[0][1]);
    xload(2 * sp + 1, dst[1][0], dst[1][1]);
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
  double xsq_part = 0.0, xsq = 0.0;
  double mx = -INFINITY;
  float sm = 0.0f;
  float run_max = -INFINITY;   // running max of the row's block maxima (running-max need bound)
  unsigned pairs = 0;

  // Component tile ct is complete: log-joint, log-sum-exp and need bounds per block.
  auto finish_tile = [&](int ct) __attribute__((always_inline)) {
    if (ct == 0) xsq = xsq_part + __shfl_xor(xsq_part, 32);
    const double2* kp0 = kc_l + (ct & 1) * CTB * 32 + g * 16;
#pragma unroll
    for (int b = 0; b < CTB; ++b) {
      const int kb = ct * CTB + b;
      if (kb < KB) {
        double ll[16];
        double bm = -INFINITY;
#pragma unroll
        for (int i = 0; i < 16; ++i) {
          const float S = ((acc[b][0][i] + acc[b][1][i]) + acc[b][2][i]) + acc[b][3][i];
          const double2 cb = kp0[b * 32 + i];
          ll[i] = fma(-cb.y, fma(-2.0, (double)S, xsq), cb.x);
          bm = fmax(bm, ll[i]);
        }
        asm volatile("" : "+v"(bm));
        const double mn = fmax(mx, bm);
        const double ms = (mn == -INFINITY) ? 0.0 : mn;
        float a = sm * fast_exp2((float)(mx - ms));
#pragma unroll
        for (int i = 0; i < 16; ++i) a += fast_exp2((float)(ll[i] - ms));
        sm = a;
        mx = mn;
        if constexpr (LJ) {
          lj_put_rows(lj + (tile * KB + kb) * kLjTile, ljmax + (tile * KB + kb) * 32, c, g, ll, bm, a, run_max,
                      dense != 0);
        } else {
          const float R = lj_row_max(bm);
          if (rexact) {
            if (g == 0) rmax_l[(wave * KB + kb) * 32 + c] = bf16_bits_up(R);
          } else {
            run_max = fmaxf(run_max, R);
            const bool nb = valid && (dense != 0 || !(R - run_max < -kLjSkipGap));
            const unsigned bits = (unsigned)__builtin_amdgcn_ballot_w64(nb);
            if (lane == 0) ljmask[tile * KB + kb] = bits;
            pairs += __builtin_popcount(bits);
          }
        }
      }
#pragma unroll
      for (int h = 0; h < kCtChains; ++h) acc[b][h] = zero16();
    }
  };

  // One stage; P = s & 1 is the LDS buffer and the register stage, and the chunks
  // 2 sp, 2 sp + 1 go to chains 2P, 2P + 1 (NS is even, so sp and s share parity).
  auto stage = [&](int ct, int sp, auto par) __attribute__((always_inline)) {
    constexpr int P = decltype(par)::value;
    const int s = ct * NS + sp;
    const bool more = s + 1 < nstage;
    if (more) fetch(s + 1);
    xstage(s + 1, xr[1 - P]);
    const bf16x8* mp = mu_l + P * SO + lane;
    bf16x8 xb[2][3];
#pragma unroll
    for (int qq = 0; qq < 2; ++qq) {
      split3_bf16(xr[P][qq][0], xr[P][qq][1], xb[qq]);
      if (ct == 0) {
#pragma unroll
        for (int e = 0; e < 4; ++e) {
          xsq_part = fma((double)xr[P][qq][0][e], (double)xr[P][qq][0][e], xsq_part);
          xsq_part = fma((double)xr[P][qq][1][e], (double)xr[P][qq][1][e], xsq_part);
        }
      }
    }
    // Block by block (its operands for both chunks), the two chunks' chains interleaved.
    // Steps in x6c_tile's order: x2 mu2, x1 mu3, x3 mu1, x2 mu1, x1 mu2, -o, x1 mu1.
#pragma unroll
    for (int b = 0; b < CTB; ++b) {
      bf16x8 a[2][4];
#pragma unroll
      for (int qq = 0; qq < 2; ++qq) {
#pragma unroll
        for (int t = 0; t < 4; ++t) a[qq][t] = mp[b * 512 + (qq * 4 + t) * 64];
      }
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
    rowstat[row] = make_double2(xsq, lz2);
    if (logZ) logZ[row] = (float)(lz2 * kLn2);
  }
  if constexpr (LJ) {
    if (g == 0) lj_put_masks(ljmax + tile * KB * 32, ljmask + tile * KB, ljcount + (tile & 63), KB, c, lz2,
                             valid, dense != 0);
  } else if (rexact) {
    const unsigned short* rm = rmax_l + wave * KB * 32 + c;
    if (g == 0)
      need_put_masks([&](int kb) { return bf16_bits_to_float(rm[kb * 32]); }, ljmask + tile * KB,
                     ljcount + (tile & 63), KB, c, lz2, valid, dense != 0);
  } else {
    const unsigned nanbits = (unsigned)__builtin_amdgcn_ballot_w64(valid && g == 0 && lz2 != lz2);
    if (lane == 0) {
      if (nanbits != 0)
        for (int kb = 0; kb < KB; ++kb) ljmask[tile * KB + kb] |= nanbits;
      if (pairs != 0) atomicAdd(ljcount + (tile & 63), pairs);
    }
  }
}

// Total of the 64 needed-pair counters (one wave, uniform result).
__device__ __forceinline__ unsigned lj_pair_total(const unsigned* __restrict__ count) {
  unsigned v = count[threadIdx.x & 63];
#pragma unroll
  for (int o = 32; o > 0; o >>= 1) v += __shfl_xor(v, o);
  return __builtin_amdgcn_readfirstlane(v);
}


// ---------------------------------------------------------------------------
// Pass 2 of the default plan (D <= 128): the log-joint is recomputed only for the
// (row, component block) pairs whose need bit pass 1 set.
//
// One wave per (row slab, component block); a workgroup holds 4 waves of one block
// on consecutive slabs, with mu of the block (bf16 splits and centring offsets,
// the B operands of x6c_tile_rows) in LDS for all four.  Each wave walks the need
// words of its slab's 32-row tiles and queues the needed rows; every 32 queued
// rows form one tile:
//   - the rows of X are loaded into registers in the A-operand layout (lane = row),
//     split three ways into bf16, and the first two splits are written row-major to
//     the wave's LDS tiles;
//   - S = X mu^T by x6c_tile_rows (lane = component, register = row), the
//     log-joint by pass 1's formula (so logZ2 and r come from one log-joint),
//     r = 2^(ll2 - logZ2), Nk and sig_acc on the VALU;
//   - r^T X on the bf16 matrix cores as r2 x1 + r1 x2 + r1 x1 (r = r1 + r2 and
//     x = x1 + x2 + x3 split exactly; the dropped terms are below 2^-16 of |r x|),
//     r as the A operand (acc_to_row_operands) and the tile's rows as the B operand
//     (lds_rows_operand, the transposing LDS read).
// The rows of the two next tiles are in flight while a tile is computed.  Workgroups are dealt
// to the 8 XCDs round-robin; the index mapping puts every component block of a
// slab group on one XCD, so a row of X that several blocks need comes from HBM
// once and from that XCD's L2 after.
// ---------------------------------------------------------------------------


__host__ __device__ constexpr size_t gather_lds_bytes(int DP) {
  return (size_t)(DP / 16) * 4 * 64 * 16                          // mu block (bf16x8 operands)
         + (size_t)kGatherWaves * 2 * 32 * gather_rs(DP) * 2      // x1, x2 tiles per wave
         + (size_t)kGatherWaves * 32 * sizeof(double2)             // row state per wave
         + (size_t)kGatherWaves * 64 * sizeof(int);                // row queue per wave
}

// Slab groups: kGatherWaves waves per workgroup, each taking spw slabs one after another.
__host__ __device__ constexpr int gather_groups(int nslab, int spw = 1) {
  return (nslab + kGatherWaves * spw - 1) / (kGatherWaves * spw);
}
__host__ inline int64_t gather_grid(int nslab, int KB, int spw = 1) {
  return gather_item_grid(gather_groups(nslab, spw), KB);
}

// Waves per SIMD of the gathering and tile passes: two where a wave's registers and
// the workgroup's LDS allow it (D <= 64), so one wave's loads and waits overlap the
// other's matrix steps.
__host__ __device__ constexpr int gather_waves_per_simd(int DP) { return DP <= 64 ? 2 : 1; }

template <int DP>
__global__ __attribute__((amdgpu_flat_work_group_size(64 * kGatherWaves, 64 * kGatherWaves),
                          amdgpu_waves_per_eu(gather_waves_per_simd(DP), gather_waves_per_simd(DP))))
void iso_accum_gather(const float* __restrict__ X, int64_t ldx, int64_t N, int D,
                      const bf16x8* __restrict__ mu3, const double4* __restrict__ kc_gat, int KB, int KP,
                      const double2* __restrict__ rowstat, const unsigned* __restrict__ need,
                      const unsigned* __restrict__ needcount, int64_t dense_min, int nslab,
                      int64_t rows_per_slab, float* __restrict__ part_mu, float* __restrict__ part_nk,
                      float* __restrict__ part_sig, int dense, ProbeSel sel, int spw) {
  constexpr int NQ = DP / 16;
  constexpr int NJ = DP / 32;
  constexpr int RS = gather_rs(DP);
  constexpr int BLK = NQ * 4 * 64;   // bf16x8 per component block
  // With at least dense_min needed rows iso_accum_tiles runs instead (uniform exit).
  if (need_total(needcount) >= dense_min) return;
  // The stored branch of FGMM_FLAG_STORE_LOGJOINT_AUTO runs instead when selected.
  if (probe_selects(sel)) return;

  extern __shared__ __align__(16) unsigned char lds_raw[];
  unsigned char* lp = lds_raw;
  bf16x8* mu_l = reinterpret_cast<bf16x8*>(lp);    lp += (size_t)BLK * sizeof(bf16x8);
  __bf16* xt_all = reinterpret_cast<__bf16*>(lp);  lp += (size_t)kGatherWaves * 2 * 32 * RS * 2;
  double2* rs_all = reinterpret_cast<double2*>(lp); lp += (size_t)kGatherWaves * 32 * sizeof(double2);
  int* q_all = reinterpret_cast<int*>(lp);

  const int tid = threadIdx.x, lane = tid & 63;
  const int wave = __builtin_amdgcn_readfirstlane(tid >> 6);
  const int c = lane & 31, g = lane >> 5;

  // Workgroup -> (slab group, block), spread over the XCDs by gather_item.  Up to
  // D = 64 (two waves per SIMD) a wave takes one slab (the host passes spw = 1).
  const int nsw = DP > 64 ? spw : 1;
  int sg, kb;
  if (!gather_item(blockIdx.x, gather_groups(nslab, nsw), KB, sg, kb)) return;   // uniform over the workgroup
  for (int idx = tid; idx < BLK; idx += 64 * kGatherWaves) mu_l[idx] = mu3[(int64_t)kb * BLK + idx];
  __syncthreads();
  // The wave's nsw slabs, one after another, each into its own partial (no barrier
  // follows).
  for (int s2 = 0; s2 < nsw; ++s2) {
  const int slab = (sg * nsw + s2) * kGatherWaves + wave;
  if (slab >= nslab) break;

  __bf16* xt = xt_all + wave * 2 * 32 * RS;   // [split][row][RS]
  double2* rs_l = rs_all + wave * 32;
  int* q_l = q_all + wave * 64;

  const double4 kc = kc_gat[(int64_t)kb * 32 + c];   // (centred C, b, ||mu||^2 - 2 sum o) of component c
  const double Cc = kc.x, bk = kc.y;
  const float mqf = (float)kc.z;

  const int64_t r_begin = (int64_t)slab * rows_per_slab;
  int64_t r_end = r_begin + rows_per_slab;
  if (r_end > N) r_end = N;
  const int64_t t_begin = r_begin / 32, t_end = cdiv(r_end, 32);

  // Need words of 64 tiles at a time, one per lane, the next batch in flight.
  auto words = [&](int64_t tb) -> unsigned {
    const int64_t t = tb + lane;
    return t < t_end ? need[t * KB + kb] : 0u;
  };
  int64_t tb = t_begin;
  unsigned mword = words(tb), mnext = words(tb + 64);
  int jn = 0;          // next word of the batch
  int qh = 0, qt = 0;  // queue head and tail (positions mod 64)

  // Queue rows until 32 are waiting (or the slab ends) and take up to 32 of them:
  // returns the count (uniform); lane c of both halves gets tile row c's offset in
  // the slab, or -1.  Rows are queued in tile order, each word's rows in bit order.
  auto take = [&](int& e) -> int {
    queue_fill<(DP > 64)>(words, tb, t_begin, t_end, mword, mnext, jn, qt, qh, lane, c, g, q_l);
    const int cnt = qt - qh < 32 ? qt - qh : 32;
    asm volatile("s_waitcnt lgkmcnt(0)" ::: "memory");
    e = c < cnt ? q_l[(qh + c) & 63] : -1;
    qh += cnt;
    return cnt;
  };

  // Rows of the tiles in flight, two deep: X in the A-operand layout and the row
  // state.  Stage P holds the tile after next while tile P is computed.
  f32x4 raw[2][2 * NQ];
  double2 rst[2];
  // The rows come through resources over the slab: a lane without a row reads zeros
  // and makes no access, and the loads of a tile issue back to back.  X so while the
  // slab spans under 2 GiB (uniform; with one offset per lane where D fills whole
  // chunks), else load_row4.
  const bool xbuf = slab_fits(r_end - r_begin, ldx);
  const bool xfull = xbuf && D == DP;
  const buf_rsrc xres = slab_rsrc(X, ldx, r_begin, xbuf ? r_end : r_begin);
  const buf_rsrc rres = make_rsrc(rowstat + r_begin, (uint32_t)((r_end - r_begin) * sizeof(double2)));
  auto issue = [&](int e, f32x4 (&rw)[2 * NQ], double2& rs) __attribute__((always_inline)) {
    const bool ok = e >= 0;
    if (xfull) {
      const int off = buf_off(ok ? (int)((int64_t)e * ldx * (int64_t)sizeof(float)) + 32 * g : kBufOob);
#pragma unroll
      for (int q = 0; q < NQ; ++q) {
        rw[2 * q] = __builtin_bit_cast(f32x4, __builtin_amdgcn_raw_buffer_load_b128(xres, off, 64 * q, 0));
        rw[2 * q + 1] = __builtin_bit_cast(f32x4, __builtin_amdgcn_raw_buffer_load_b128(xres, off, 64 * q + 16, 0));
      }
    } else if (xbuf) {
#pragma unroll
      for (int q = 0; q < NQ; ++q) {
        rw[2 * q] = slab_row4(xres, ldx, e, 16 * q + 8 * g, D, ok);
        rw[2 * q + 1] = slab_row4(xres, ldx, e, 16 * q + 8 * g + 4, D, ok);
      }
    } else {
      const int64_t row = r_begin + (ok ? e : 0);
#pragma unroll
      for (int q = 0; q < NQ; ++q) {
        rw[2 * q] = load_row4(X, ldx, row, 16 * q + 8 * g, D, ok);
        rw[2 * q + 1] = load_row4(X, ldx, row, 16 * q + 8 * g + 4, D, ok);
      }
    }
    const double2 v = __builtin_bit_cast(
        double2, __builtin_amdgcn_raw_buffer_load_b128(rres, buf_off(ok ? e * (int)sizeof(double2) : kBufOob), 0, 0));
    rs = make_double2(v.x, ok ? v.y : INFINITY);   // a row past the queue: logZ2 = +inf, r = 0
  };

  f32x16 acc[NJ];
#pragma unroll
  for (int j = 0; j < NJ; ++j) acc[j] = zero16();
  float nk = 0.0f, sig = 0.0f;
  const bf16x8 ones = x6c_ones(lane);

  // One tile from stage P; the tile two ahead is taken from the queue and its loads
  // issued into the same stage once its registers are free.  Returns that tile's count.
  auto tile = [&](auto par) __attribute__((always_inline)) -> int {
    constexpr int P = decltype(par)::value;
    // This tile's rows: bf16 splits in registers, x1 and x2 to LDS, row state to LDS.
    bf16x8 xa[NQ][3];
#pragma unroll
    for (int q = 0; q < NQ; ++q) split3_bf16(raw[P][2 * q], raw[P][2 * q + 1], xa[q]);
    asm volatile("s_waitcnt lgkmcnt(0)" ::: "memory");   // the previous tile's LDS reads are done
#pragma unroll
    for (int q = 0; q < NQ; ++q) {
#pragma unroll
      for (int sp = 0; sp < 2; ++sp)
        *reinterpret_cast<bf16x8*>(xt + (sp * 32 + c) * RS + 16 * q + 8 * g) = xa[q][sp];
    }
    if (g == 0) rs_l[c] = rst[P];
    int en;
    const int cnt_ahead = take(en);
    if (cnt_ahead > 0) issue(en, raw[P], rst[P]);
    asm volatile("s_waitcnt lgkmcnt(0)" ::: "memory");

    const f32x16 S = x6c_tile_rows<NQ, kIsoChains>(xa, ones, [&](int q, int t) { return mu_l[(q * 4 + t) * 64 + lane]; });
    float r[16], res[16];
#pragma unroll
    for (int i = 0; i < 16; ++i) {
      const double2 w = rs_l[acc_row(i, g)];   // (||x||^2, logZ2) of the row
      const double ll = fma(-bk, fma(-2.0, (double)S[i], w.x), Cc);
      const float rv = fast_exp2((float)(ll - w.y));
      r[i] = rv;
      res[i] = rv - (float)(__bf16)rv;
      nk += rv;
      sig = fmaf(rv, fmaf(-2.0f, S[i], (float)w.x) + mqf, sig);
    }
    bf16x8 a1[2], a2[2];
    acc_to_row_operands(r, a1);
    acc_to_row_operands(res, a2);
#pragma unroll
    for (int p = 0; p < 2; ++p) {
      // A step whose responsibilities all round to zero adds nothing (their residuals
      // are zero too): skipped, with identical results.
      if (dense || any_nonzero(a1[p])) {
#pragma unroll
        for (int j = 0; j < NJ; ++j) {
          const bf16x8 b1 = lds_rows_operand(xt, RS, 16 * p, 32 * j, lane);
          const bf16x8 b2 = lds_rows_operand(xt + 32 * RS, RS, 16 * p, 32 * j, lane);
          acc[j] = mfma_bf16(a2[p], b1, acc[j]);
          acc[j] = mfma_bf16(a1[p], b2, acc[j]);
          acc[j] = mfma_bf16(a1[p], b1, acc[j]);
        }
      }
    }
    return cnt_ahead;
  };

  int e;
  int cnt0 = take(e);
  if (cnt0 > 0) issue(e, raw[0], rst[0]);
  int cnt1 = cnt0 > 0 ? take(e) : 0;
  if (cnt1 > 0) issue(e, raw[1], rst[1]);
  while (cnt0 > 0) {
    cnt0 = tile(std::integral_constant<int, 0>{});
    if (cnt1 == 0) break;
    cnt1 = tile(std::integral_constant<int, 1>{});
  }

  nk += __shfl_xor(nk, 32);
  sig += __shfl_xor(sig, 32);
  const int64_t kbase = (int64_t)slab * KP + (int64_t)kb * 32;
#pragma unroll
  for (int j = 0; j < NJ; ++j) {
#pragma unroll
    for (int i = 0; i < 16; ++i) part_mu[(kbase + acc_row(i, g)) * DP + 32 * j + c] = acc[j][i];
  }
  if (g == 0) {
    part_nk[kbase + c] = nk;
    part_sig[kbase + c] = sig;
  }
  }
}


// ---------------------------------------------------------------------------
// Pass 2 of the default plan (D <= 64; iso_accum_tiles2 at D = 96 and 128) when
// most pairs are needed (pass 1 counted at least dense_min needed rows; the
// gathering kernel runs otherwise).  Grid over (row slab x group of 4 component
// blocks), two waves per SIMD; wave w owns block
// 4 cg + w, its mu operands in registers, and the slab's partial of that block
// (the gathering kernel's slab split, so either kernel fills the same partials).
// The 32-row tiles of X are loaded once per workgroup, split three ways into bf16
// by all 256 threads and kept row-major in LDS (double-buffered), where the four
// waves read the A operands of S (x6c_tile_rows) and the transposed B operands of
// r^T X (lds_rows_operand).  A wave whose need word of the tile is zero skips it;
// rows whose bit is clear enter with responsibilities that are exactly zero.
// ---------------------------------------------------------------------------
constexpr int kTileBlocks = 4;

__host__ __device__ constexpr size_t tiles_lds_bytes(int DP) {
  return (size_t)2 * 3 * 32 * gather_rs(DP) * 2 + (size_t)2 * 32 * sizeof(double2);
}

template <int DP>
__global__ __attribute__((amdgpu_flat_work_group_size(64 * kTileBlocks, 64 * kTileBlocks),
                          amdgpu_waves_per_eu(gather_waves_per_simd(DP), gather_waves_per_simd(DP))))
void iso_accum_tiles(const float* __restrict__ X, int64_t ldx, int64_t N, int D,
                     const bf16x8* __restrict__ mu3, const double4* __restrict__ kc_gat, int KB, int KP,
                     const double2* __restrict__ rowstat, const unsigned* __restrict__ need,
                     const unsigned* __restrict__ needcount, int64_t dense_min, int nslab,
                     int64_t rows_per_slab, float* __restrict__ part_mu, float* __restrict__ part_nk,
                     float* __restrict__ part_sig, int dense, ProbeSel sel) {
  constexpr int NQ = DP / 16;
  constexpr int NJ = DP / 32;
  constexpr int RS = gather_rs(DP);
  constexpr int BLK = NQ * 4 * 64;
  constexpr int NT = 64 * kTileBlocks;
  constexpr int V4 = DP / 4;              // float4 per row
  constexpr int LPT = 32 * V4 / NT;       // float4 per thread per tile
  static_assert((32 * V4) % NT == 0, "tile split");
  if (need_total(needcount) < dense_min) return;   // the gathering kernel runs (uniform exit)
  if (probe_selects(sel)) return;   // the stored branch runs

  extern __shared__ __align__(16) unsigned char lds_raw[];
  __bf16* xs = reinterpret_cast<__bf16*>(lds_raw);                                   // [2][3][32][RS]
  double2* rs_l = reinterpret_cast<double2*>(lds_raw + (size_t)2 * 3 * 32 * RS * 2);  // [2][32]

  const int tid = threadIdx.x, lane = tid & 63;
  const int wave = __builtin_amdgcn_readfirstlane(tid >> 6);
  const int c = lane & 31, g = lane >> 5;
  const int slab = (int)(blockIdx.x % (unsigned)nslab);
  const int kb = (int)(blockIdx.x / (unsigned)nslab) * kTileBlocks + wave;
  const bool active = kb < KB;

  bf16x8 mb[NQ][4];
#pragma unroll
  for (int q = 0; q < NQ; ++q) {
#pragma unroll
    for (int t = 0; t < 4; ++t) {
      bf16x8 z;
#pragma unroll
      for (int e = 0; e < 8; ++e) z[e] = (__bf16)0.0f;
      mb[q][t] = active ? mu3[(int64_t)kb * BLK + (q * 4 + t) * 64 + lane] : z;
    }
  }
  double Cc = -INFINITY, bk = 0.0;
  float mqf = 0.0f;
  if (active) {
    const double4 kc = kc_gat[(int64_t)kb * 32 + c];
    Cc = kc.x; bk = kc.y; mqf = (float)kc.z;
  }

  const int64_t r_begin = (int64_t)slab * rows_per_slab;
  int64_t r_end = r_begin + rows_per_slab;
  if (r_end > N) r_end = N;
  const int64_t t_begin = r_begin / 32, t_end = r_end > r_begin ? cdiv(r_end, 32) : t_begin;

  f32x4 st[LPT];
  double2 rst = make_double2(0.0, INFINITY);
  // Tile rows through a resource over the slab (no branch per load, rows past the
  // slab read zeros) while it spans under 2 GiB (uniform), else load_row4.
  const bool xbuf = slab_fits(r_end - r_begin, ldx);
  const buf_rsrc xres = slab_rsrc(X, ldx, r_begin, xbuf ? r_end : r_begin);
  auto fetch = [&](int64_t t) {
    const int64_t row0 = t * 32;
#pragma unroll
    for (int u = 0; u < LPT; ++u) {
      const int idx = u * NT + tid;
      const int64_t row = row0 + idx / V4;
      const int d0 = (idx % V4) * 4;
      st[u] = xbuf ? slab_row4(xres, ldx, (int)(row - r_begin), d0, D, row < r_end)
                   : load_row4(X, ldx, row, d0, D, row < r_end);
    }
    if (tid < 32) {
      const int64_t row = row0 + tid;
      rst = row < r_end ? rowstat[row] : make_double2(0.0, INFINITY);
    }
  };
  // Split the staged tile into bf16 x1, x2, x3 (4 values per float4: two packed pairs).
  auto commit = [&](int buf) {
    __bf16* dst = xs + (size_t)buf * 3 * 32 * RS;
#pragma unroll
    for (int u = 0; u < LPT; ++u) {
      const int idx = u * NT + tid;
      const int rr = idx / V4, d0 = (idx % V4) * 4;
      uint2 w[3];
#pragma unroll
      for (int j = 0; j < 2; ++j) {
        const f32x2 a = {st[u][2 * j], st[u][2 * j + 1]};
        const unsigned h = bf16_pair(a);
        const f32x2 r = a - bf16_pair_widen(h);
        const unsigned m = bf16_pair(r);
        const unsigned l = bf16_pair(r - bf16_pair_widen(m));
        (j == 0 ? w[0].x : w[0].y) = h;
        (j == 0 ? w[1].x : w[1].y) = m;
        (j == 0 ? w[2].x : w[2].y) = l;
      }
#pragma unroll
      for (int sp = 0; sp < 3; ++sp) *reinterpret_cast<uint2*>(dst + (sp * 32 + rr) * RS + d0) = w[sp];
    }
    if (tid < 32) rs_l[buf * 32 + tid] = rst;
  };

  f32x16 acc[NJ];
#pragma unroll
  for (int j = 0; j < NJ; ++j) acc[j] = zero16();
  float nk = 0.0f, sig = 0.0f;
  const bf16x8 ones = x6c_ones(lane);

  if (t_begin < t_end) {
    fetch(t_begin);
    commit(0);
  }
  __syncthreads();
  // The tile's need word, loaded one tile ahead (a load used at once would stall every tile).
  auto need_of = [&](int64_t t) -> unsigned { return active ? (dense ? ~0u : need[t * KB + kb]) : 0u; };
  unsigned mnext = t_begin < t_end ? need_of(t_begin) : 0u;
  for (int64_t t = t_begin; t < t_end; ++t) {
    const int buf = (int)((t - t_begin) & 1);
    const bool more = t + 1 < t_end;
    if (more) fetch(t + 1);
    const unsigned m = mnext;
    if (more) mnext = need_of(t + 1);
    if (m != 0u) {
      const __bf16* xt = xs + (size_t)buf * 3 * 32 * RS;
      bf16x8 xa[NQ][3];
#pragma unroll
      for (int q = 0; q < NQ; ++q) {
#pragma unroll
        for (int sp = 0; sp < 3; ++sp)
          xa[q][sp] = *reinterpret_cast<const bf16x8*>(xt + (sp * 32 + c) * RS + 16 * q + 8 * g);
      }
      const f32x16 S = x6c_tile_rows<NQ, kIsoChains>(xa, ones, [&](int q, int t4) { return mb[q][t4]; });
      const double2* rw = rs_l + buf * 32;
      float r[16], res[16];
#pragma unroll
      for (int i = 0; i < 16; ++i) {
        const double2 w = rw[acc_row(i, g)];
        const double ll = fma(-bk, fma(-2.0, (double)S[i], w.x), Cc);
        const float rv = fast_exp2((float)(ll - w.y));
        r[i] = rv;
        res[i] = rv - (float)(__bf16)rv;
        nk += rv;
        sig = fmaf(rv, fmaf(-2.0f, S[i], (float)w.x) + mqf, sig);
      }
      bf16x8 a1[2], a2[2];
      acc_to_row_operands(r, a1);
      acc_to_row_operands(res, a2);
#pragma unroll
      for (int p = 0; p < 2; ++p) {
        if (dense || any_nonzero(a1[p])) {
#pragma unroll
          for (int j = 0; j < NJ; ++j) {
            const bf16x8 b1 = lds_rows_operand(xt, RS, 16 * p, 32 * j, lane);
            const bf16x8 b2 = lds_rows_operand(xt + 32 * RS, RS, 16 * p, 32 * j, lane);
            acc[j] = mfma_bf16(a2[p], b1, acc[j]);
            acc[j] = mfma_bf16(a1[p], b2, acc[j]);
            acc[j] = mfma_bf16(a1[p], b1, acc[j]);
          }
        }
      }
    }
    if (more) commit(buf ^ 1);
    __syncthreads();
  }

  if (active) {
    nk += __shfl_xor(nk, 32);
    sig += __shfl_xor(sig, 32);
    const int64_t kbase = (int64_t)slab * KP + (int64_t)kb * 32;
#pragma unroll
    for (int j = 0; j < NJ; ++j) {
#pragma unroll
      for (int i = 0; i < 16; ++i) part_mu[(kbase + acc_row(i, g)) * DP + 32 * j + c] = acc[j][i];
    }
    if (g == 0) {
      part_nk[kbase + c] = nk;
      part_sig[kbase + c] = sig;
    }
  }
}

// ---------------------------------------------------------------------------
// The tile pass for D = 96 and 128, where a wave holding a block's mu operands for
// all of D leaves room for one wave per SIMD only: each block is split over two
// waves by accumulation chain.  Eight waves per workgroup; wave (h, w) owns block
// 4 cg + w and chain h, that is the chunks q = h, h + 2, ... (the chunks pass 1's
// chain h adds, in the same order), so it keeps half the operands.  Per 32-row tile:
//   - each wave forms its chain over the tile's rows (x6c_tile_rows' products and
//     order) and leaves it in LDS; after a barrier both waves of a block add the two
//     chains as pass 1 does, c0 + c1, and have S bit for bit;
//   - wave (h, w) takes the 16 rows of step h (registers 8h .. 8h + 7 of S): their
//     log-joint, r and residual, Nk and sig_acc, and their r^T X for all of D;
//   - at the end the two waves' partials of a block are added in a fixed order.
// Two waves per SIMD, so the waits of one overlap the other's matrix steps.  The X
// tiles are triple-buffered and the chain exchange double-buffered, so one barrier
// per tile orders everything: tile t + 2 is written after it, into the buffer that
// tile t - 1 left, which every wave finished before the barrier.
// ---------------------------------------------------------------------------
constexpr int kTileWaves2 = 2 * kTileBlocks;

__host__ __device__ constexpr size_t tiles2_lds_bytes(int DP) {
  return (size_t)3 * 3 * 32 * gather_rs(DP) * 2 + (size_t)3 * 32 * sizeof(double2) +
         (size_t)2 * kTileWaves2 * 4 * 64 * sizeof(f32x4);
}

template <int DP>
__global__ __attribute__((amdgpu_flat_work_group_size(64 * kTileWaves2, 64 * kTileWaves2),
                          amdgpu_waves_per_eu(2, 2)))
void iso_accum_tiles2(const float* __restrict__ X, int64_t ldx, int64_t N, int D,
                      const bf16x8* __restrict__ mu3, const double4* __restrict__ kc_gat, int KB, int KP,
                      const double2* __restrict__ rowstat, const unsigned* __restrict__ need,
                      const unsigned* __restrict__ needcount, int64_t dense_min, int nslab,
                      int64_t rows_per_slab, float* __restrict__ part_mu, float* __restrict__ part_nk,
                      float* __restrict__ part_sig, int dense, ProbeSel sel) {
  constexpr int NQ = DP / 16;
  constexpr int NQH = NQ / 2;              // chunks of this wave's chain
  constexpr int NJ = DP / 32;
  constexpr int RS = gather_rs(DP);
  constexpr int BLK = NQ * 4 * 64;
  constexpr int NT = 64 * kTileWaves2;
  constexpr int V4 = DP / 4;               // float4 per row
  constexpr int NV = 32 * V4;              // float4 per tile
  constexpr int LPT = (NV + NT - 1) / NT;  // float4 per thread per tile
  static_assert(NQ % 2 == 0 && kIsoChains == 2, "one chain per wave of a pair");
  if (need_total(needcount) < dense_min) return;   // the gathering kernel runs (uniform exit)
  if (probe_selects(sel)) return;   // the stored branch runs

  extern __shared__ __align__(16) unsigned char lds_raw[];
  __bf16* xs = reinterpret_cast<__bf16*>(lds_raw);                                   // [3][3][32][RS]
  double2* rs_l = reinterpret_cast<double2*>(lds_raw + (size_t)3 * 3 * 32 * RS * 2);  // [3][32]
  f32x4* ex = reinterpret_cast<f32x4*>(rs_l + 3 * 32);                                // [2][wave][4][64]

  const int tid = threadIdx.x, lane = tid & 63;
  const int wave = __builtin_amdgcn_readfirstlane(tid >> 6);
  const int w = wave % kTileBlocks, h = wave / kTileBlocks;
  const int c = lane & 31, g = lane >> 5;
  const int slab = (int)(blockIdx.x % (unsigned)nslab);
  const int kb = (int)(blockIdx.x / (unsigned)nslab) * kTileBlocks + w;
  const bool active = kb < KB;

  // This wave's chain: operands of the chunks q = 2u + h.
  bf16x8 mb[NQH][4];
#pragma unroll
  for (int u = 0; u < NQH; ++u) {
#pragma unroll
    for (int t = 0; t < 4; ++t) {
      bf16x8 z;
#pragma unroll
      for (int e = 0; e < 8; ++e) z[e] = (__bf16)0.0f;
      mb[u][t] = active ? mu3[(int64_t)kb * BLK + ((2 * u + h) * 4 + t) * 64 + lane] : z;
    }
  }
  double Cc = -INFINITY, bk = 0.0;
  float mqf = 0.0f;
  if (active) {
    const double4 kc = kc_gat[(int64_t)kb * 32 + c];
    Cc = kc.x; bk = kc.y; mqf = (float)kc.z;
  }

  const int64_t r_begin = (int64_t)slab * rows_per_slab;
  int64_t r_end = r_begin + rows_per_slab;
  if (r_end > N) r_end = N;
  const int64_t t_begin = r_begin / 32, t_end = r_end > r_begin ? cdiv(r_end, 32) : t_begin;

  f32x4 st[LPT];
  double2 rst = make_double2(0.0, INFINITY);
  // Tile rows through a resource over the slab (no branch per load, rows past the
  // slab read zeros) while it spans under 2 GiB (uniform), else load_row4.
  const bool xbuf = slab_fits(r_end - r_begin, ldx);
  const buf_rsrc xres = slab_rsrc(X, ldx, r_begin, xbuf ? r_end : r_begin);
  auto fetch = [&](int64_t t) {
    const int64_t row0 = t * 32;
#pragma unroll
    for (int u = 0; u < LPT; ++u) {
      const int idx = u * NT + tid;
      const int64_t row = row0 + (idx < NV ? idx / V4 : 0);
      const int d0 = (idx % V4) * 4;
      const bool ok = idx < NV && row < r_end;
      st[u] = xbuf ? slab_row4(xres, ldx, (int)(row - r_begin), d0, D, ok) : load_row4(X, ldx, row, d0, D, ok);
    }
    if (tid < 32) {
      const int64_t row = row0 + tid;
      const double2 z = rowstat[row < r_end ? row : r_begin];   // a row of the slab: no branch
      rst = row < r_end ? z : make_double2(0.0, INFINITY);
    }
  };
  // Split the staged tile into bf16 x1, x2, x3 (4 values per float4: two packed pairs).
  auto commit = [&](int buf) {
    __bf16* dst = xs + (size_t)buf * 3 * 32 * RS;
#pragma unroll
    for (int u = 0; u < LPT; ++u) {
      const int idx = u * NT + tid;
      if (NV % NT != 0 && idx >= NV) continue;
      const int rr = idx / V4, d0 = (idx % V4) * 4;
      uint2 wd[3];
#pragma unroll
      for (int j = 0; j < 2; ++j) {
        const f32x2 a = {st[u][2 * j], st[u][2 * j + 1]};
        const unsigned hi = bf16_pair(a);
        const f32x2 r = a - bf16_pair_widen(hi);
        const unsigned m = bf16_pair(r);
        const unsigned l = bf16_pair(r - bf16_pair_widen(m));
        (j == 0 ? wd[0].x : wd[0].y) = hi;
        (j == 0 ? wd[1].x : wd[1].y) = m;
        (j == 0 ? wd[2].x : wd[2].y) = l;
      }
#pragma unroll
      for (int sp = 0; sp < 3; ++sp) *reinterpret_cast<uint2*>(dst + (sp * 32 + rr) * RS + d0) = wd[sp];
    }
    if (tid < 32) rs_l[buf * 32 + tid] = rst;
  };

  f32x16 acc[NJ];
#pragma unroll
  for (int j = 0; j < NJ; ++j) acc[j] = zero16();
  float nk = 0.0f, sig = 0.0f;
  const bf16x8 ones = x6c_ones(lane);
  constexpr int EXB = kTileWaves2 * 4 * 64;                         // f32x4 per exchange buffer

  for (int p = 0; p < 2; ++p) {
    if (t_begin + p < t_end) {
      fetch(t_begin + p);
      commit(p);
    }
  }
  __syncthreads();
  // The tile's need word (the same for both waves of a block), loaded one tile ahead.
  auto need_of = [&](int64_t t) -> unsigned { return active ? (dense ? ~0u : need[t * KB + kb]) : 0u; };
  unsigned mnext = t_begin < t_end ? need_of(t_begin) : 0u;
  for (int64_t t = t_begin; t < t_end; ++t) {
    const int it = (int)(t - t_begin);
    const int buf = it % 3;
    const bool more = t + 2 < t_end;
    if (more) fetch(t + 2);
    const unsigned m = mnext;
    if (t + 1 < t_end) mnext = need_of(t + 1);
    const __bf16* xt = xs + (size_t)buf * 3 * 32 * RS;
    f32x4* mine = ex + (it & 1) * EXB + wave * 4 * 64 + lane;
    const f32x4* ch0 = ex + (it & 1) * EXB + w * 4 * 64 + lane;                   // chain 0 of the block
    const f32x4* ch1 = ex + (it & 1) * EXB + (kTileBlocks + w) * 4 * 64 + lane;   // chain 1
    if (m != 0u) {
      // Chain h over the tile's rows: x6c_tile_rows' steps for the chunks q = 2u + h.
      f32x16 cacc = zero16();
#pragma unroll
      for (int u = 0; u < NQH; ++u) {
        const int q = 2 * u + h;
        bf16x8 xa[3];
#pragma unroll
        for (int sp = 0; sp < 3; ++sp) xa[sp] = *reinterpret_cast<const bf16x8*>(xt + (sp * 32 + c) * RS + 16 * q + 8 * g);
        cacc = mfma_bf16(xa[1], mb[u][1], cacc);
        cacc = mfma_bf16(xa[0], mb[u][2], cacc);
        cacc = mfma_bf16(xa[2], mb[u][0], cacc);
        cacc = mfma_bf16(xa[1], mb[u][0], cacc);
        cacc = mfma_bf16(xa[0], mb[u][1], cacc);
        cacc = mfma_bf16(ones, mb[u][3], cacc);
        cacc = mfma_bf16(xa[0], mb[u][0], cacc);
      }
#pragma unroll
      for (int k = 0; k < 4; ++k) mine[k * 64] = f32x4{cacc[4 * k], cacc[4 * k + 1], cacc[4 * k + 2], cacc[4 * k + 3]};
    }
    __syncthreads();   // both chains of every block are in LDS
    if (m != 0u) {
      // Registers 8h .. 8h + 7 of S = c0 + c1: the rows of step h.
      float S[8];
#pragma unroll
      for (int k = 0; k < 2; ++k) {
        const f32x4 a = ch0[(2 * h + k) * 64], b = ch1[(2 * h + k) * 64];
        S[4 * k] = a.x + b.x; S[4 * k + 1] = a.y + b.y; S[4 * k + 2] = a.z + b.z; S[4 * k + 3] = a.w + b.w;
      }
      const double2* rw = rs_l + buf * 32;
      float r[8], res[8];
#pragma unroll
      for (int k = 0; k < 8; ++k) {
        const double2 z = rw[acc_row(8 * h + k, g)];
        const double ll = fma(-bk, fma(-2.0, (double)S[k], z.x), Cc);
        const float rv = fast_exp2((float)(ll - z.y));
        r[k] = rv;
        res[k] = rv - (float)(__bf16)rv;
        nk += rv;
        sig = fmaf(rv, fmaf(-2.0f, S[k], (float)z.x) + mqf, sig);
      }
      const bf16x8 a1 = acc_to_row_operand(r), a2 = acc_to_row_operand(res);
      if (dense || any_nonzero(a1)) {
#pragma unroll
        for (int j = 0; j < NJ; ++j) {
          const bf16x8 b1 = lds_rows_operand(xt, RS, 16 * h, 32 * j, lane);
          const bf16x8 b2 = lds_rows_operand(xt + 32 * RS, RS, 16 * h, 32 * j, lane);
          acc[j] = mfma_bf16(a2, b1, acc[j]);
          acc[j] = mfma_bf16(a1, b2, acc[j]);
          acc[j] = mfma_bf16(a1, b1, acc[j]);
        }
      }
    }
    if (more) commit((it + 2) % 3);
  }
  __syncthreads();   // the last tile's exchange has been read

  // The two waves' partials of a block, added in a fixed order (h = 0 first) by wave
  // (0, w) through LDS, one 32-column tile at a time.
  nk += __shfl_xor(nk, 32);
  sig += __shfl_xor(sig, 32);
  const int64_t kbase = (int64_t)slab * KP + (int64_t)kb * 32;
  float* exf = reinterpret_cast<float*>(ex);
#pragma unroll
  for (int j = 0; j < NJ; ++j) {
    if (h == 1) {
#pragma unroll
      for (int i = 0; i < 16; ++i) exf[(w * 16 + i) * 64 + lane] = acc[j][i];
      if (j == 0) {
        exf[(kTileBlocks * 16) * 64 + w * 64 + lane] = nk;
        exf[(kTileBlocks * 16 + kTileBlocks) * 64 + w * 64 + lane] = sig;
      }
    }
    __syncthreads();
    if (h == 0 && active) {
#pragma unroll
      for (int i = 0; i < 16; ++i)
        part_mu[(kbase + acc_row(i, g)) * DP + 32 * j + c] = acc[j][i] + exf[(w * 16 + i) * 64 + lane];
      if (j == 0 && g == 0) {
        part_nk[kbase + c] = nk + exf[(kTileBlocks * 16) * 64 + w * 64 + lane];
        part_sig[kbase + c] = sig + exf[(kTileBlocks * 16 + kTileBlocks) * 64 + w * 64 + lane];
      }
    }
    __syncthreads();
  }
}

// ---------------------------------------------------------------------------
// Pass 2 of the default plan above D = 128.  One workgroup of four waves per (row
// slab, component block, range of up to kDrange dimensions).  The waves walk the
// slab's need words alike, so they queue the same rows; for every 32 queued rows:
//   - wave w forms chain w of S = X mu^T, the chunks q = w, w + 4, ... of all of D
//     with x6c_tile_rows' products and order (mu's operands read from global
//     memory), and writes the first two bf16 splits of those of its chunks that lie
//     in the workgroup's range to the LDS tile of the rows;
//   - the four chains meet in LDS and every wave adds them as pass 1 does,
//     ((c0 + c1) + c2) + c3, so S, the log-joint and r equal pass 1's bit for bit;
//   - r = 2^(ll2 - logZ2), and wave w accumulates r^T X for its quarter of the
//     range's 32-column tiles (r2 x1 + r1 x2 + r1 x1, the rows read transposed from
//     LDS); wave 0 of the first range also sums Nk and sig_acc.
// Wider D runs several ranges, each workgroup recomputing S.  Workgroups are dealt
// to the XCDs so that each XCD serves a contiguous run of component blocks: at this
// width mu of a block is the larger operand stream, and it stays in that XCD's L2.
// ---------------------------------------------------------------------------
__global__ __attribute__((amdgpu_flat_work_group_size(64 * kCtWaves, 64 * kCtWaves), amdgpu_waves_per_eu(1, 1)))
void iso_accum_drange(const float* __restrict__ X, int64_t ldx, int64_t N, int D, int NQ, int DP,
                      const bf16x8* __restrict__ mu3, const double4* __restrict__ kc_gat, int KB, int KP,
                      const double2* __restrict__ rowstat, const unsigned* __restrict__ need, int nslab,
                      int64_t rows_per_slab, int ndr, float* __restrict__ part_mu, float* __restrict__ part_nk,
                      float* __restrict__ part_sig, int dense) {
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
  __bf16* xt = reinterpret_cast<__bf16*>(lp);     lp += (size_t)2 * 32 * RS * 2;   // [split][row][RS]
  float* ex = reinterpret_cast<float*>(lp);       lp += (size_t)kCtWaves * 16 * 64 * sizeof(float);
  double2* rs_l = reinterpret_cast<double2*>(lp); lp += (size_t)32 * sizeof(double2);
  int* q_all = reinterpret_cast<int*>(lp);

  const int tid = threadIdx.x, lane = tid & 63;
  const int wave = __builtin_amdgcn_readfirstlane(tid >> 6);
  const int c = lane & 31, g = lane >> 5;
  int* q_l = q_all + wave * 64;

  const int d0 = dr * kDrange;
  const int DR = DP - d0 < kDrange ? DP - d0 : kDrange;   // a multiple of 64
  const int q_lo = d0 / 16, q_hi = (d0 + DR) / 16;         // chunks of the range
  const int njr = DR / 32;
  const int tj = (njr + kCtWaves - 1) / kCtWaves;
  const int j0 = wave * tj;
  const int nj = njr - j0 < tj ? (njr - j0 > 0 ? njr - j0 : 0) : tj;   // this wave's column tiles
  const int nqw = NQ / kCtWaves;                                       // chunks per wave (NQ % 4 == 0)

  const double4 kc = kc_gat[(int64_t)kb * 32 + c];   // (centred C, b, ||mu||^2 - 2 sum o) of component c
  const double Cc = kc.x, bk = kc.y;
  const float mqf = (float)kc.z;

  const int64_t r_begin = (int64_t)slab * rows_per_slab;
  int64_t r_end = r_begin + rows_per_slab;
  if (r_end > N) r_end = N;
  const int64_t t_begin = r_begin / 32, t_end = cdiv(r_end, 32);

  // Need words of 64 tiles at a time, one per lane, the next batch in flight.
  auto words = [&](int64_t tb) -> unsigned {
    const int64_t t = tb + lane;
    return t < t_end ? need[t * KB + kb] : 0u;
  };
  int64_t tb = t_begin;
  unsigned mword = words(tb), mnext = words(tb + 64);
  int jn = 0;          // next word of the batch
  int qh = 0, qt = 0;  // queue head and tail (positions mod 64)
  // Queue rows until 32 are waiting (or the slab ends) and take up to 32 of them:
  // returns the count (the same in every wave); lane c of both halves gets tile row
  // c's offset in the slab, or -1.
  auto take = [&](int& e) -> int {
    queue_fill<true>(words, tb, t_begin, t_end, mword, mnext, jn, qt, qh, lane, c, g, q_l);
    const int cnt = qt - qh < 32 ? qt - qh : 32;
    asm volatile("s_waitcnt lgkmcnt(0)" ::: "memory");
    e = c < cnt ? q_l[(qh + c) & 63] : -1;
    qh += cnt;
    return cnt;
  };

  // Chunk i of this wave (chunk q = wave + 4 i): the rows' dimensions 16q + 8g .. + 7
  // and mu's four operands of the chunk.
  const buf_rsrc mrs = make_rsrc(mu3 + (int64_t)kb * NQ * 4 * 64, (uint32_t)((int64_t)NQ * 4 * 64 * sizeof(bf16x8)));
  auto issue = [&](int i, int e, f32x4 (&x)[2], bf16x8 (&m)[4]) {
    const int q = wave + kCtWaves * i;
    const bool ok = e >= 0;
    const int64_t row = r_begin + (ok ? e : 0);
    x[0] = load_row4(X, ldx, row, 16 * q + 8 * g, D, ok);
    x[1] = load_row4(X, ldx, row, 16 * q + 8 * g + 4, D, ok);
#pragma unroll
    for (int t = 0; t < 4; ++t)
      m[t] = __builtin_bit_cast(bf16x8, __builtin_amdgcn_raw_buffer_load_b128(
                                            mrs, lane * (int)sizeof(bf16x8), (q * 4 + t) * 64 * (int)sizeof(bf16x8), 0));
  };
  f32x4 xr[2][2];
  bf16x8 mr[2][4];
  double2 rst = make_double2(0.0, INFINITY);
  auto start = [&](int e) {
    issue(0, e, xr[0], mr[0]);
    if (nqw > 1) issue(1, e, xr[1], mr[1]);
    if (wave == 0) {
      const double2 z = rowstat[r_begin + (e >= 0 ? e : 0)];   // a row of the slab: no branch
      rst = e >= 0 ? z : make_double2(0.0, INFINITY);
    }
  };

  f32x16 acc[kDrTiles];
#pragma unroll
  for (int j = 0; j < kDrTiles; ++j) acc[j] = zero16();
  float nk = 0.0f, sig = 0.0f;
  const bf16x8 ones = x6c_ones(lane);

  int e;
  int cnt = take(e);
  if (cnt > 0) start(e);
  while (cnt > 0) {
    // Chain `wave` of S over this wave's chunks (x6c_tile_rows' steps per chunk).
    f32x16 cs = zero16();
    auto chunk = [&](int i, const f32x4 (&x)[2], const bf16x8 (&m)[4]) {
      const int q = wave + kCtWaves * i;
      bf16x8 xa[3];
      split3_bf16(x[0], x[1], xa);
      if (q >= q_lo && q < q_hi) {
#pragma unroll
        for (int sp = 0; sp < 2; ++sp)
          *reinterpret_cast<bf16x8*>(xt + (sp * 32 + c) * RS + 16 * (q - q_lo) + 8 * g) = xa[sp];
      }
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
    // The next rows: queued now, their first chunks in flight during r^T X.
    int en;
    const int cnt_next = take(en);
    if (cnt_next > 0) start(en);
    lds_barrier();

    float r[16], res[16];
#pragma unroll
    for (int i = 0; i < 16; ++i) {
      const float S = ((ex[i * 64 + lane] + ex[(16 + i) * 64 + lane]) + ex[(32 + i) * 64 + lane]) +
                      ex[(48 + i) * 64 + lane];
      const double2 w = rs_l[acc_row(i, g)];   // (||x||^2, logZ2) of the row
      const double ll = fma(-bk, fma(-2.0, (double)S, w.x), Cc);
      const float rv = fast_exp2((float)(ll - w.y));
      r[i] = rv;
      res[i] = rv - (float)(__bf16)rv;
      nk += rv;
      sig = fmaf(rv, fmaf(-2.0f, S, (float)w.x) + mqf, sig);
    }
    bf16x8 a1[2], a2[2];
    acc_to_row_operands(r, a1);
    acc_to_row_operands(res, a2);
#pragma unroll
    for (int p = 0; p < 2; ++p) {
      if (dense || any_nonzero(a1[p])) {
#pragma unroll
        for (int jj = 0; jj < kDrTiles; ++jj) {
          if (jj < nj) {
            const int col = 32 * (j0 + jj);
            const bf16x8 b1 = lds_rows_operand(xt, RS, 16 * p, col, lane);
            const bf16x8 b2 = lds_rows_operand(xt + 32 * RS, RS, 16 * p, col, lane);
            acc[jj] = mfma_bf16(a2[p], b1, acc[jj]);
            acc[jj] = mfma_bf16(a1[p], b2, acc[jj]);
            acc[jj] = mfma_bf16(a1[p], b1, acc[jj]);
          }
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
      for (int i = 0; i < 16; ++i)
        part_mu[(kbase + acc_row(i, g)) * DP + d0 + 32 * (j0 + jj) + c] = acc[jj][i];
    }
  }
  if (dr == 0 && wave == 0) {
    nk += __shfl_xor(nk, 32);
    sig += __shfl_xor(sig, 32);
    if (g == 0) {
      part_nk[kbase + c] = nk;
      part_sig[kbase + c] = sig;
    }
  }
}

// ---------------------------------------------------------------------------
// Pass 2 from the stored log-joint: grid over (row slab x group of CB component
// blocks); eight waves = CB component blocks x NH column parts x 8 / (CB NH) row
// groups of 32 rows (NH = 2 above D = 128, where one wave's accumulators for all
// of D would not fit in registers).  Each wave reads the log-joint rows of its
// block that pass 1 marked as needed (a 128-byte line per row), forms
// r = 2^(ll2 - logZ2) and accumulates r^T X for its columns on the matrix cores
// from the X tile that the workgroup's blocks share in LDS.  ||x - mu_k||^2 for
// sig_acc comes back from the log-joint as (C0_k - ll2) / b_k, where
// C0_k = C_k + b_k ||mu_k||^2.  logZ2 sits in LDS as a hi + lo pair of floats, so
// ll2 - logZ2 keeps the accuracy of the fp32 log-joint.
//
// Streaming, with NB register buffers (3 up to D = 128, else 2 for registers):
// while tile t is processed, X super-tile t + NB and the log-joint rows of tile
// t + NB - 1 are loaded, so each has NB - 1 iterations or more to arrive.  The need
// masks that select those rows travel with X: super-tile u carries the masks of
// tile u + NB - 1.  The loop is unrolled by NB so that every register buffer has a fixed
// index (no copies between iterations), and every load is a range-checked buffer
// load issued unconditionally, so the compiler waits only for the loads each
// instruction consumes.
// ---------------------------------------------------------------------------
__host__ __device__ constexpr int accum_lj_buffers(int DP) { return DP <= 128 ? 3 : 2; }

template <int DP, int CB, int NH>
constexpr size_t accum_lj_lds_bytes() {
  return (size_t)2 * 32 * (kAccWaves / (CB * NH)) * ((DP + 4) * sizeof(float) + sizeof(float2)) +
         (size_t)2 * kAccWaves * sizeof(unsigned);
}

template <int DP, int CB, int NH>
__global__ __attribute__((amdgpu_flat_work_group_size(kAccThreads, kAccThreads), amdgpu_waves_per_eu(2, 2)))
void iso_accum_lj(const float* __restrict__ X, int64_t ldx, int64_t N, int D,
                  const float* __restrict__ lj, const unsigned* __restrict__ ljmask,
                  const unsigned* __restrict__ ljcount, int64_t sparse_max,
                  const double4* __restrict__ kc_lin, int KB, int KP,
                  const double2* __restrict__ rowstat, int nslab, int64_t rows_per_slab,
                  float* __restrict__ part_mu, float* __restrict__ part_nk, float* __restrict__ part_sig,
                  int dense) {
  constexpr int NJ = DP / 32 / NH;               // 32-column accumulator tiles per wave
  constexpr int RS = DP + 4;
  constexpr int V4 = DP / 4;
  constexpr int RG = kAccWaves / (CB * NH);      // row groups (32 rows each)
  constexpr int TR = 32 * RG;                    // rows per super-tile
  constexpr int NV = TR * V4;                    // float4 per super-tile
  constexpr int LPT = (NV + kAccThreads - 1) / kAccThreads;
  static_assert(kAccWaves % (CB * NH) == 0 && (DP / 32) % NH == 0, "even split");
  static_assert(TR + kAccWaves <= kAccThreads, "row-state and mask threads");

  // iso_accum_sparse takes the call when pass 1 found the masks sparse.
  if (sparse_max >= 0 && (int64_t)lj_pair_total(ljcount) <= sparse_max) return;

  extern __shared__ __align__(16) unsigned char lds_raw[];
  float* xs = reinterpret_cast<float*>(lds_raw);                                  // [2][TR*RS]
  float2* rz = reinterpret_cast<float2*>(lds_raw + 2 * TR * RS * sizeof(float));  // [2][TR]
  unsigned* mk = reinterpret_cast<unsigned*>(rz + 2 * TR);                        // [2][kAccWaves]

  const int tid = threadIdx.x, lane = tid & 63;
  const int wave = __builtin_amdgcn_readfirstlane(tid >> 6);
  const int c = lane & 31, g = lane >> 5;
  const int cbw = wave % CB, h = (wave / CB) % NH, rg = wave / (CB * NH);
  const int slab = blockIdx.x % nslab;
  const int cg = blockIdx.x / nslab;
  const int kb = cg * CB + cbw;
  const bool active = kb < KB;
  const int col0 = h * (DP / NH);                 // first column of this wave's part

  const int64_t r_begin = (int64_t)slab * rows_per_slab;
  int64_t r_end = r_begin + rows_per_slab;
  if (r_end > N) r_end = N;
  const int ntiles = r_end > r_begin ? (int)cdiv(r_end - r_begin, TR) : 0;

  // C0_k and 1 / b_k; zero for padding and for components with log_pi = -inf
  // (their r is 0, and the clamp below keeps 0 * inf out of sig).
  float c0 = 0.0f, ibk = 0.0f;
  if (active) {
    const double4 kc = kc_lin[(int64_t)kb * 32 + c];
    const double c0d = fma(kc.y, kc.z, kc.x);
    if (c0d > -INFINITY && c0d < INFINITY) {
      c0 = (float)c0d;
      ibk = (float)(1.0 / kc.y);
    }
  }

  f32x16 acc[NJ];
#pragma unroll
  for (int j = 0; j < NJ; ++j) acc[j] = zero16();
  float nk = 0.0f, sig = 0.0f;

  // Need mask of (row tile, block): bit r set when row r of the 32-row tile may
  // have a nonzero responsibility in the block; 0 past the slab or the blocks.
  const buf_rsrc mask_r = make_rsrc(ljmask, (uint32_t)(cdiv(N, 32) * KB * sizeof(unsigned)));
  auto mask_off = [&](int t, int rgw, int kbw) -> int {
    const int64_t row0 = r_begin + (int64_t)t * TR + rgw * 32;
    return (t < ntiles && row0 < r_end && kbw < KB) ? (int)(((row0 >> 5) * KB + kbw) * 4) : kBufOob;
  };

  constexpr int NB = accum_lj_buffers(DP);

  // Super-tile t: X rows, their logZ2 (threads < TR) and the need masks of tile
  // t + NB - 1 (thread TR + w for wave w), which the waves read once tile t is in
  // LDS.  Rows past the slab, columns past D and tiles past the end read as zero.
  const bool ragged = (D & 3) != 0;
  auto fetch = [&](int t, f32x4 (&st)[LPT], double& rqv, unsigned& mqv) {
    const int64_t row0 = r_begin + (int64_t)t * TR;
    int nrow = 0;
    if (t < ntiles) nrow = (int)(r_end - row0 < TR ? r_end - row0 : TR);
    const buf_rsrc xr = make_rsrc(nrow ? X + row0 * ldx : X, (uint32_t)(nrow * ldx * 4));
#pragma unroll
    for (int q = 0; q < LPT; ++q) {
      const int idx = q * kAccThreads + tid;
      const int r = idx / V4, col = (idx % V4) * 4;
      const bool ok = (NV % kAccThreads == 0 || idx < NV) && r < nrow && col < D;
      st[q] = buf_load_f32x4(xr, ok ? (int)((r * ldx + col) * 4) : kBufOob);
    }
    const buf_rsrc rr = make_rsrc(nrow ? rowstat + row0 : rowstat, (uint32_t)(nrow * sizeof(double2)));
    const double q2 = buf_load_f64(rr, tid < nrow ? tid * (int)sizeof(double2) + 8 : kBufOob);
    rqv = tid < nrow ? q2 : INFINITY;   // rows past the slab: logZ2 = +inf, hence r = 0
    const int w = tid - TR;
    mqv = buf_load_u32(mask_r, (w >= 0 && w < kAccWaves)
                                   ? mask_off(t + NB - 1, w / (CB * NH), cg * CB + w % CB)
                                   : kBufOob);
  };
  // Columns past D within the last float4 of a row are zeroed here, where the
  // loaded values are consumed anyway.
  auto commit = [&](int buf, const f32x4 (&st)[LPT], double rqv, unsigned mqv) {
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
  // Log-joint rows of tile t (register i: rows 8 (i >> 2) + (i & 3) + 4g), those
  // whose need bit is set; the others read as 0.
  auto lj_fetch = [&](int t, unsigned m, f32x16& v) {
    const int64_t row0 = r_begin + (int64_t)t * TR + rg * 32;
    const buf_rsrc lr = make_rsrc(m ? lj + ((row0 >> 5) * KB + kb) * kLjTile : lj, m ? kLjTile * 4 : 0);
#pragma unroll
    for (int i = 0; i < 16; ++i) {
      const int row = 8 * (i >> 2) + (i & 3) + 4 * g;
      v[i] = buf_load_f32<kBufNt>(lr, ((m >> row) & 1u) ? (row * 32 + c) * 4 : kBufOob);
    }
  };

  f32x4 stg[NB][LPT];
  double rqs[NB];
  unsigned mqs[NB];
  f32x16 ljb[NB];
  // Need masks of tiles t .. t + NB - 2 (msk[0] is the current tile's).
  unsigned msk[NB - 1];

  // One tile; P = t mod NB.  Registers P receive X super-tile t + NB (free since
  // tile t went to LDS), log-joint buffer (P + NB - 1) mod NB tile t + NB - 1 (free
  // since tile t - 1 was processed); X tile t + 1 goes from registers (P + 1) mod NB
  // to the other LDS buffer at the end.
  auto step = [&](int t, auto par) {
    constexpr int P = decltype(par)::value;
    const int lb = t & 1;   // LDS buffer of tile t
    const unsigned ma = __builtin_amdgcn_readfirstlane(mk[lb * kAccWaves + wave]);   // tile t + NB - 1
    lj_fetch(t + NB - 1, ma, ljb[(P + NB - 1) % NB]);
    fetch(t + NB, stg[P], rqs[P], mqs[P]);
    const unsigned mc = msk[0];
    const float* xt = xs + lb * TR * RS + rg * 32 * RS;
    const float2* rt = rz + lb * TR + rg * 32 + 4 * g;
    if (active && mc != 0u) {
      const float* xbase = xt + 4 * g * RS + col0 + c;
      // Register rows i whose need bits (rows 8q + j and 8q + j + 4 for i = 4q + j)
      // are not both clear, in ascending order: r = 2^(ll2 - logZ2) for the lanes
      // whose row is needed, 0 for the others (their log-joint was not read), then
      // one matrix-core step per 32 columns unless every r is zero.  The skipped rows
      // have r = 0 on every lane, so the sums are those of the dense order.
      unsigned pm = (mc | (mc >> 4)) & 0x0f0f0f0fu;
      const unsigned mg = mc >> (4 * g);
      if (__builtin_popcount(pm) >= 8) {
        // A dense tile: all 16 register rows unrolled, in the same order.
#pragma unroll
        for (int q = 0; q < 4; ++q) {
          const f32x4 z01 = *reinterpret_cast<const f32x4*>(rt + 8 * q);
          const f32x4 z23 = *reinterpret_cast<const f32x4*>(rt + 8 * q + 2);
          const float zh[4] = {z01.x, z01.z, z23.x, z23.z}, zl[4] = {z01.y, z01.w, z23.y, z23.w};
#pragma unroll
          for (int j = 0; j < 4; ++j) {
            const int ro = 8 * q + j;
            if ((pm >> ro) & 1u) {
              const float l = ljb[P][4 * q + j];
              const float rv = ((mg >> ro) & 1u) ? fast_exp2((l - zh[j]) - zl[j]) : 0.0f;
              if (NH == 1 || h == 0) {
                nk += rv;
                sig = fmaf(rv, c0 - l, sig);
              }
              if (dense || __builtin_amdgcn_ballot_w64(rv != 0.0f) != 0) {
#pragma unroll
                for (int jj = 0; jj < NJ; ++jj) acc[jj] = mfma32(rv, xbase[ro * RS + 32 * jj], acc[jj]);
              }
            }
          }
        }
        pm = 0u;
      }
      // Two register rows per round (the second optional), their LDS reads issued
      // together so that the two latency chains overlap.
      while (pm != 0u) {
        const int ro0 = __builtin_ctz(pm);   // 8q + j
        pm &= pm - 1u;
        const bool two = pm != 0u;
        const int ro1 = two ? __builtin_ctz(pm) : ro0;
        if (two) pm &= pm - 1u;
        const float2 z0 = rt[ro0], z1 = rt[ro1];
        float xo0[NJ], xo1[NJ];
#pragma unroll
        for (int jj = 0; jj < NJ; ++jj) {
          xo0[jj] = xbase[ro0 * RS + 32 * jj];
          xo1[jj] = xbase[ro1 * RS + 32 * jj];
        }
        const float l0 = ljb[P][4 * (ro0 >> 3) + (ro0 & 3)];
        const float l1 = ljb[P][4 * (ro1 >> 3) + (ro1 & 3)];
        const float rv0 = ((mg >> ro0) & 1u) ? fast_exp2((l0 - z0.x) - z0.y) : 0.0f;
        const float rv1 = (two && ((mg >> ro1) & 1u)) ? fast_exp2((l1 - z1.x) - z1.y) : 0.0f;
        if (NH == 1 || h == 0) {
          // sig gathers r (C0_k - ll2) = r b_k ||x - mu_k||^2; 1 / b_k is applied once
          // at the end (a component of weight 0 has ll2 = -inf there, so its lane's
          // sum turns NaN and is dropped below).  Rows not read have l = 0, r = 0.
          nk += rv0;
          sig = fmaf(rv0, c0 - l0, sig);
          if (two) {
            nk += rv1;
            sig = fmaf(rv1, c0 - l1, sig);
          }
        }
        if (dense || __builtin_amdgcn_ballot_w64(rv0 != 0.0f) != 0) {
#pragma unroll
          for (int jj = 0; jj < NJ; ++jj) acc[jj] = mfma32(rv0, xo0[jj], acc[jj]);
        }
        if (two && (dense || __builtin_amdgcn_ballot_w64(rv1 != 0.0f) != 0)) {
#pragma unroll
          for (int jj = 0; jj < NJ; ++jj) acc[jj] = mfma32(rv1, xo1[jj], acc[jj]);
        }
      }
    }
    if (t + 1 < ntiles) commit(lb ^ 1, stg[(P + 1) % NB], rqs[(P + 1) % NB], mqs[(P + 1) % NB]);
    lds_barrier();
#pragma unroll
    for (int u = 0; u + 1 < NB - 1; ++u) msk[u] = msk[u + 1];
    msk[NB - 2] = ma;
  };

  if (ntiles > 0) {
#pragma unroll
    for (int u = 0; u < NB; ++u) fetch(u, stg[u], rqs[u], mqs[u]);
#pragma unroll
    for (int u = 0; u < NB - 1; ++u) {
      msk[u] = __builtin_amdgcn_readfirstlane(buf_load_u32(mask_r, mask_off(u, rg, kb)));
      lj_fetch(u, msk[u], ljb[u]);
    }
    commit(0, stg[0], rqs[0], mqs[0]);
    lds_barrier();
  }
  using P0 = std::integral_constant<int, 0>;
  using P1 = std::integral_constant<int, 1>;
  using P2 = std::integral_constant<int, 2>;
  for (int t = 0; t < ntiles; t += NB) {
    step(t, P0{});
    if (t + 1 >= ntiles) break;
    step(t + 1, P1{});
    if constexpr (NB == 3) {
      if (t + 2 >= ntiles) break;
      step(t + 2, P2{});
    }
  }

  if (active) {
    nk += __shfl_xor(nk, 32);
    sig += __shfl_xor(sig, 32);
    sig = ibk != 0.0f ? sig * ibk : 0.0f;
    const int64_t kbase = ((int64_t)slab * RG + rg) * KP + (int64_t)kb * 32;
#pragma unroll
    for (int j = 0; j < NJ; ++j) {
#pragma unroll
      for (int i = 0; i < 16; ++i)
        part_mu[(kbase + acc_row(i, g)) * DP + col0 + 32 * j + c] = acc[j][i];
    }
    if (g == 0 && h == 0) {
      part_nk[kbase + c] = nk;
      part_sig[kbase + c] = sig;
    }
  }
}

// ---------------------------------------------------------------------------
// Pass 2 from the stored log-joint up to D = 128.  Pass 1 (iso_lse_pipe storing)
// leaves per 32-row tile the log-joint of every block, the bf16 (hi, lo) parts of
// the tile's X rows (row-major at this kernel's LDS row stride) and the rows' logZ2
// as (hi, lo) float pairs.  r^T X runs on the bf16 matrix cores in the split form of
// the gathering pass: r and x each in two bf16 parts and, per 16-row step, the
// products r2 x1, r1 x2 and r1 x1 added in that order.
//
// Grid over (row slab x group of kLjtWaves = 4 component blocks); wave w owns block
// 4 cg + w and that block's partial of the slab.  The workgroups of a slab are dealt
// to one XCD, so that the X parts come from HBM once and from that XCD's L2 for the
// other groups.  Two LDS stages, each one tile's X parts, the 4 blocks' log-joint
// tiles and the logZ2 pairs, all filled by buffer-to-LDS loads: at step t the
// workgroup issues tile t + 1's, computes tile t and waits for tile t + 1's before
// the barrier.  Two such workgroups share a compute unit (one wave of each per
// SIMD), so one computes while the other waits at its barrier: with one 8-wave
// workgroup of three stages the waves spent 37% of their cycles waiting (1.32 ms at
// N=1M, K=1024, D=128 on N(0, I) data; 1.20 ms this way).
// A wave issues the same loads every step, so that wait is a fixed count of its own
// outstanding loads, and no global load of the loop is left for the compiler to
// wait on.  A wave skips a tile whose need word is zero (its loads then read out of
// range); otherwise it loads and exponentiates the whole log-joint tile with no
// per-row select: a row whose need bit is clear has l < logZ2 - kLjNeedGap in every
// component of the block, so 2^(l - logZ2) is exactly 0 in fp32, and pass 1 gives a
// row past N the logZ2 pair (+inf, 0).  `sel` (when given) is the word pass 1 read:
// the kernel returns unless set.
// ---------------------------------------------------------------------------
constexpr int kLjtWaves = kLjtWavesPlan;
constexpr int kLjtStages = 2;

template <int DP>
struct LjtShape {
  static constexpr int XB = (int)ljt_xsplit_bytes(DP);     // a tile's X parts
  static constexpr int XP = XB / 16;                        // their 16-byte pieces, a multiple of 64
  static constexpr int XQ = (XP + 64 * kLjtWaves - 1) / (64 * kLjtWaves);
  static constexpr int LJB = kLjtWaves * kLjTile * 4;       // the blocks' log-joint tiles
  static constexpr int OFF_X = LJB, OFF_Z = LJB + XB;
  static constexpr int STAGE = LJB + XB + 32 * 8;
  // After the stages, one 1 KB line that the loads a wave issues only to keep its
  // count fixed (out of range: they write zeros) land in.
  static constexpr int OFF_PAD = kLjtStages * STAGE;
  static constexpr size_t lds = (size_t)OFF_PAD + 1024;
  // Loads of every wave per tile: XQ of X parts (the last one out of range on the
  // waves past XP), 4 of its log-joint tile, 1 of logZ2 pairs (wave 0; an
  // out-of-range one elsewhere).
  static constexpr int NLOADS = XQ + 4 + 1;
};
__host__ inline int64_t ljt_grid(int nslab, int ncg) { return (int64_t)8 * cdiv(nslab, 8) * ncg; }


template <int DP>
__global__ __attribute__((amdgpu_flat_work_group_size(64 * kLjtWaves, 64 * kLjtWaves), amdgpu_waves_per_eu(2, 2)))
void iso_accum_ljt(const float* __restrict__ lj, const __bf16* __restrict__ xsplit, const float2* __restrict__ zpair,
                   int64_t N, const unsigned* __restrict__ ljmask, const unsigned* __restrict__ ljcount,
                   int64_t sparse_max, ProbeSel sel, const double4* __restrict__ kc_lin,
                   int KB, int KP, int nslab, int64_t rows_per_slab, int ncg, float* __restrict__ part_mu,
                   float* __restrict__ part_nk, float* __restrict__ part_sig, int dense) {
  static_assert(DP <= 128 && DP % 32 == 0, "one 32-row tile of X per stage");
  using SH = LjtShape<DP>;
  static_assert(SH::XP % 64 == 0, "whole waves of X pieces");
  constexpr int NJ = DP / 32;
  constexpr int RS = gather_rs(DP);
  constexpr int NS = kLjtStages;
  // iso_accum_sparse takes the call when pass 1 found the masks sparse; with a
  // selector word, the recomputing kernels take it unless the word is set.
  if (sparse_max >= 0 && need_total(ljcount) <= sparse_max) return;
  if (sel.count != nullptr && !probe_selects(sel)) return;

  extern __shared__ __align__(16) unsigned char lds_raw[];

  const int tid = threadIdx.x, lane = tid & 63;
  const int wave = __builtin_amdgcn_readfirstlane(tid >> 6);
  const int c = lane & 31, g = lane >> 5;
  // Workgroup -> (slab, component group): the ncg groups of slab s run on XCD s % 8.
  const int xcd = blockIdx.x & 7, item = blockIdx.x >> 3;
  const int slab = (item / ncg) * 8 + xcd, cg = item % ncg;
  if (slab >= nslab) return;   // uniform over the workgroup
  const int kb = cg * kLjtWaves + wave;
  const bool active = kb < KB;

  const int64_t r_begin = (int64_t)slab * rows_per_slab;
  int64_t r_end = r_begin + rows_per_slab;
  if (r_end > N) r_end = N;
  const int ntiles = r_end > r_begin ? (int)cdiv(r_end - r_begin, 32) : 0;
  const int64_t tile0 = r_begin >> 5;   // rows_per_slab is a multiple of 32

  // C0_k and 1 / b_k, as iso_accum_lj forms them.
  float c0 = 0.0f, ibk = 0.0f;
  if (active) {
    const double4 kc = kc_lin[(int64_t)kb * 32 + c];
    const double c0d = fma(kc.y, kc.z, kc.x);
    if (c0d > -INFINITY && c0d < INFINITY) {
      c0 = (float)c0d;
      ibk = (float)(1.0 / kc.y);
    }
  }
  f32x16 acc[NJ];
#pragma unroll
  for (int j = 0; j < NJ; ++j) acc[j] = zero16();
  float nk = 0.0f, sig = 0.0f;

  // The wave's need word of tile t (0 past the slab or the blocks): a scalar load.
  auto mword = [&](int t) -> unsigned {
    const bool ok = active && t < ntiles;
    const unsigned v = ljmask[ok ? (tile0 + t) * KB + kb : 0];
    return ok ? v : 0u;
  };
  // Tile t into stage S: the X parts (whole waves of pieces), the wave's log-joint
  // tile (piece l of load q is row 8 q + l / 8; all out of range when the need word
  // is 0 or the tile is past the slab) and, by wave 0, the rows' logZ2 pairs.
  constexpr int NL = SH::NLOADS;
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
      if (q * 64 * kLjtWaves + wave * 64 < SH::XP)
        lds_dma16(xsrc, st + SH::OFF_X + (q * 64 * kLjtWaves + wave * 64) * 16,
                  (q * 64 * kLjtWaves + tid) * 16, 0);
      else
        lds_dma16(xsrc, pad, kBufOob, 0);
    }
    const DmaSrc lsrc = dma_src(m ? lj + (tg * KB + kb) * kLjTile : lj, m ? (uint32_t)(kLjTile * 4) : 0u);
#pragma unroll
    for (int q = 0; q < 4; ++q) lds_dma16(lsrc, st + wave * kLjTile * 4 + q * 1024, (q * 64 + lane) * 16, 0);
    if (wave == 0) {
      // All 32 pairs of a tile in range (those of rows past N are (+inf, 0)).
      const DmaSrc zsrc = dma_src(zpair + tg * 32 * (in ? 1 : 0), in ? (uint32_t)(32 * sizeof(float2)) : 0u);
      if (lane < 16) lds_dma16(zsrc, st + SH::OFF_Z, lane * 16, 0);
    } else {
      lds_dma16(lsrc, pad, kBufOob, 0);
    }
  };
  // Tile t in stage S (need word m, not 0): one straight-line block, its LDS reads
  // issued ahead of their uses, half 1's reads and VALU work issued while half 0's
  // matrix steps run.  (The stage base goes through a register, so that the reads
  // keep small offsets.)
  auto compute = [&](auto stage_tag, unsigned m) __attribute__((always_inline)) {
    constexpr int S = decltype(stage_tag)::value;
    int sb = S * SH::STAGE;
    asm volatile("" : "+s"(sb));
    const unsigned char* st = lds_raw + sb;
    // The lane's column of rows 4g, 4g + 1, ... of the wave's log-joint tile and its
    // logZ2 pairs, each from one base register and immediate offsets.
    int lofs = sb + wave * kLjTile * 4 + 4 * c + 4 * 32 * 4 * g;
    int zofs = sb + SH::OFF_Z + 4 * 8 * g;
    asm volatile("" : "+v"(lofs), "+v"(zofs));
    const float* lt = reinterpret_cast<const float*>(lds_raw + lofs);
    const f32x4* zt = reinterpret_cast<const f32x4*>(lds_raw + zofs);
    const __bf16* xt = reinterpret_cast<const __bf16*>(st + SH::OFF_X);
    float lv[16];
    float2 zv[16];
    // Registers 4j .. 4j + 3 hold rows 8j + 4g .. 8j + 4g + 3 (acc_row).
    auto rows = [&](int p) __attribute__((always_inline)) {
#pragma unroll
      for (int jj = 0; jj < 2; ++jj) {
        const int j = 2 * p + jj;
#pragma unroll
        for (int e = 0; e < 4; ++e) lv[4 * j + e] = lt[(8 * j + e) * 32];
        const f32x4 z01 = zt[4 * j], z23 = zt[4 * j + 1];
        zv[4 * j] = make_float2(z01[0], z01[1]);
        zv[4 * j + 1] = make_float2(z01[2], z01[3]);
        zv[4 * j + 2] = make_float2(z23[0], z23[1]);
        zv[4 * j + 3] = make_float2(z23[2], z23[3]);
      }
    };
    bf16x8 b1[2][NJ], b2[2][NJ];
    auto bops = [&](int p) __attribute__((always_inline)) {
#pragma unroll
      for (int j = 0; j < NJ; ++j) {
        b1[p][j] = lds_rows_operand(xt, RS, 16 * p, 32 * j, lane);
        b2[p][j] = lds_rows_operand(xt + 32 * RS, RS, 16 * p, 32 * j, lane);
      }
    };
    bf16x8 a1[2], a2[2];
    // Responsibilities of rows 16 p .. 16 p + 15 (registers 8 p .. 8 p + 7 of the
    // accumulator layout) and their bf16 (hi, lo) parts, each pair rounded once.
    auto half = [&](int p) __attribute__((always_inline)) {
      float r[8];
#pragma unroll
      for (int e = 0; e < 8; ++e) {
        const int i = 8 * p + e;
        const float l = lv[i];
        const float rv = fast_exp2((l - zv[i].x) - zv[i].y);
        r[e] = rv;
        nk += rv;
        sig = fmaf(rv, c0 - l, sig);
      }
      acc_to_row_operands_split(r, a1[p], a2[p]);
    };
    auto steps = [&](int p) __attribute__((always_inline)) {
#pragma unroll
      for (int j = 0; j < NJ; ++j) {
        acc[j] = mfma_bf16(a2[p], b1[p][j], acc[j]);
        acc[j] = mfma_bf16(a1[p], b2[p][j], acc[j]);
        acc[j] = mfma_bf16(a1[p], b1[p][j], acc[j]);
      }
    };
    // All of the tile's LDS reads first, then half 0's responsibilities; half 1's
    // VALU work is interleaved with half 0's matrix steps (one step, then about an
    // NJ-th of the work: the wave issues it while the matrix core runs the step).
    rows(0);
    bops(0);
    rows(1);
    bops(1);
    half(0);
    __builtin_amdgcn_sched_barrier(0);
    steps(0);
    half(1);
#pragma unroll
    for (int k = 0; k < 3 * NJ; ++k) {
      __builtin_amdgcn_sched_group_barrier(0x008, 1, 0);
      __builtin_amdgcn_sched_group_barrier(0x002, 24 / NJ, 0);
    }
    __builtin_amdgcn_sched_barrier(0);
    steps(1);
  };

  unsigned mk[NS];   // need words of the tiles in the stages
  unsigned mnext = 0u;
  // Step t, stage S = t mod NS: issue tile t + NS - 1 (its stage was freed by the
  // last barrier), compute tile t, wait for tile t + 1's stage (the loads issued
  // after it are those of tiles t + 2 ..), barrier.
  auto step = [&](int t, auto stage_tag) __attribute__((always_inline)) {
    constexpr int S = decltype(stage_tag)::value;
    constexpr int SI = (S + NS - 1) % NS;
    mk[SI] = mnext;
    issue(t + NS - 1, std::integral_constant<int, SI>{}, mnext);
    mnext = mword(t + NS);
    if (mk[S] != 0u) compute(stage_tag, mk[S]);
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
    sig += __shfl_xor(sig, 32);
    sig = ibk != 0.0f ? sig * ibk : 0.0f;
    const int64_t kbase = (int64_t)slab * KP + (int64_t)kb * 32;
#pragma unroll
    for (int j = 0; j < NJ; ++j) {
#pragma unroll
      for (int i = 0; i < 16; ++i) part_mu[(kbase + acc_row(i, g)) * DP + 32 * j + c] = acc[j][i];
    }
    if (g == 0) {
      part_nk[kbase + c] = nk;
      part_sig[kbase + c] = sig;
    }
  }
}

// ---------------------------------------------------------------------------
// Pass 2 from the sparse stored log-joint, for data whose need masks are sparse
// (clustered data: most (row, block) pairs have no nonzero responsibility).  No
// workgroup-wide staging: each wave owns one (row slab, row group, component
// block), the same split as iso_accum_lj, and walks its 32-row tiles in the same
// order, so it writes the same partials bit for bit.  Per tile it fetches only the
// register-row pairs (rows r and r + 4) with a need bit: their log-joint, logZ2 and
// X rows, straight from memory into registers.
//
// The first kSparseSlots pairs of a tile have fixed register slots and are loaded
// kSparseDepth tiles ahead; every slot load is issued whether or not the slot is
// used (range-checked buffer loads, out of range when unused), so the compiler
// waits only for the slots each tile consumes.  Further pairs of a tile are loaded
// when the tile is processed.  The masks of 256 tiles at a time are staged in LDS.
//
// The accumulator tile jj holds columns NJ * c + jj (lane c), so that each lane
// reads its NJ columns of an X row with one load; every sum is formed in the same
// order as in iso_accum_lj (pairs in ascending row order, unread rows r = 0), and
// both kernels run on every call: each returns at once unless the needed-pair
// count of pass 1 selects it.
// ---------------------------------------------------------------------------
constexpr int kSparseSlots = 3;
constexpr int kSparseDepth = 4;
constexpr int kSparseBatch = 256;
constexpr int kSparseWaves = 4;

template <int DP>
__global__ __launch_bounds__(64 * kSparseWaves)
void iso_accum_sparse(const float* __restrict__ X, int64_t ldx, int64_t N, const float* __restrict__ lj,
                      const unsigned* __restrict__ ljmask, const unsigned* __restrict__ ljcount,
                      int64_t sparse_max, const double4* __restrict__ kc_lin, int KB, int KP,
                      const double2* __restrict__ rowstat, int nslab, int RG, int64_t rows_per_slab,
                      float* __restrict__ part_mu, float* __restrict__ part_nk,
                      float* __restrict__ part_sig, int dense) {
  constexpr int NJ = DP / 32;
  constexpr int S = kSparseSlots;
  constexpr int PD = kSparseDepth;
  constexpr int BT = kSparseBatch;
  typedef float fNJ __attribute__((ext_vector_type(NJ)));
  // The batch's tiles with a nonzero mask, in order: (mask, tile offset in the batch).
  __shared__ uint2 work[kSparseWaves][BT];

  if (need_total(ljcount) > sparse_max) return;
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

  float c0 = 0.0f, ibk = 0.0f;
  {
    const double4 kc = kc_lin[(int64_t)kb * 32 + c];
    const double c0d = fma(kc.y, kc.z, kc.x);
    if (c0d > -INFINITY && c0d < INFINITY) {
      c0 = (float)c0d;
      ibk = (float)(1.0 / kc.y);
    }
  }
  f32x16 acc[NJ];
#pragma unroll
  for (int j = 0; j < NJ; ++j) acc[j] = zero16();
  float nk = 0.0f, sig = 0.0f;

  // One window per tile for each operand: the tile's log-joint (4 KiB), its rows'
  // state and its X rows (32 rows; rows past N are never in range, their need bits
  // being clear).
  const int64_t row00 = r_begin + rg * 32;
  const float* lj0 = lj + ((row00 >> 5) * KB + kb) * kLjTile;
  const double2* rs0 = rowstat + row00;
  const float* x0 = X + row00 * ldx;
  const int64_t lj_step = (int64_t)RG * KB * kLjTile, x_step = TR * ldx;
  auto windows = [&](int t, buf_rsrc& lr, buf_rsrc& rr, buf_rsrc& xr) {
    lr = make_rsrc(lj0 + t * lj_step, kLjTile * 4);
    rr = make_rsrc(rs0 + (int64_t)t * TR, 32 * sizeof(double2));
    xr = make_rsrc(x0 + t * x_step, (uint32_t)(32 * ldx * 4));
  };

  // Slot registers of the PD tiles in flight.
  float sl[PD][S];
  double sz[PD][S];
  fNJ sx[PD][S];
  unsigned smk[PD];
  int stl[PD];

  // Loads of one register-row pair (rows ro and ro + 4; this lane's is ro + 4g) of
  // tile t; nothing when `used` is false or this lane's row is not needed.
  auto load_pair = [&](const buf_rsrc& lr, const buf_rsrc& rr, const buf_rsrc& xr, unsigned m, int ro,
                       bool used, float& l, double& z, fNJ& x) {
    const int row = ro + 4 * g;
    const bool need = used && ((m >> row) & 1u);
    l = buf_load_f32<kBufNt>(lr, buf_off(need ? (row * 32 + c) * 4 : kBufOob));
    z = buf_load_f64(rr, buf_off(need ? row * (int)sizeof(double2) + 8 : kBufOob));
    const int xo = buf_off(need ? (int)((row * ldx + NJ * c) * 4) : kBufOob);
    if constexpr (NJ == 4) {
      x = buf_load_f32x4(xr, xo);
    } else if constexpr (NJ == 3) {
      x = __builtin_bit_cast(fNJ, __builtin_amdgcn_raw_buffer_load_b96(xr, xo, 0, 0));
    } else {
      x = __builtin_bit_cast(fNJ, __builtin_amdgcn_raw_buffer_load_b64(xr, xo, 0, 0));
    }
  };
  // One pair's contribution, in the arithmetic of iso_accum_lj.
  auto accumulate = [&](unsigned m, int ro, float l, double q, const fNJ& x) {
    const bool need = (m >> (ro + 4 * g)) & 1u;
    const float zh = (float)q;
    const float zl = (q > -INFINITY && q < INFINITY) ? (float)(q - (double)zh) : 0.0f;
    const float rv = need ? fast_exp2((l - zh) - zl) : 0.0f;
    nk += rv;
    sig = fmaf(rv, c0 - l, sig);
    if (dense || __builtin_amdgcn_ballot_w64(rv != 0.0f) != 0) {
#pragma unroll
      for (int jj = 0; jj < NJ; ++jj) acc[jj] = mfma32(rv, x[jj], acc[jj]);
    }
  };
  // Issue work item k of the batch (tile b0 + offset) into stage u; past the count,
  // mask 0 makes every load out of range.
  auto issue = [&](int k, int cnt, int b0, int u) {
    unsigned m = 0u;
    int t = 0;
    if (k < cnt) {
      const uint2 e = work[wave][k];
      m = __builtin_amdgcn_readfirstlane(e.x);
      t = b0 + __builtin_amdgcn_readfirstlane(e.y);
    }
    smk[u] = m;
    stl[u] = t;
    buf_rsrc lr, rr, xr;
    windows(t, lr, rr, xr);
    unsigned pm = lj_pair_mask(m);
#pragma unroll
    for (int j = 0; j < S; ++j) {
      const bool used = pm != 0u;
      const int ro = used ? __builtin_ctz(pm) : 0;
      pm &= pm - 1u;
      load_pair(lr, rr, xr, m, ro, used, sl[u][j], sz[u][j], sx[u][j]);
    }
  };
  auto process = [&](int u) {
    const unsigned m = smk[u];
    if (m == 0u) return;
    unsigned pm = lj_pair_mask(m);
#pragma unroll
    for (int j = 0; j < S; ++j) {
      if (pm == 0u) return;
      const int ro = __builtin_ctz(pm);
      pm &= pm - 1u;
      accumulate(m, ro, sl[u][j], sz[u][j], sx[u][j]);
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
      load_pair(lr, rr, xr, m, ro, true, l, q, x);
      accumulate(m, ro, l, q, x);
    }
  };

  for (int b0 = 0; b0 < ntiles; b0 += BT) {
    // Compact the batch's nonzero masks (this wave only; LDS is in order per wave).
    int cnt = 0;
#pragma unroll
    for (int q = 0; q < BT / 64; ++q) {
      const int t = b0 + 64 * q + lane;
      const int64_t row0 = r_begin + (int64_t)t * TR + rg * 32;
      const unsigned m = (t < ntiles && row0 < r_end) ? ljmask[(row0 >> 5) * KB + kb] : 0u;
      const unsigned long long bal = __builtin_amdgcn_ballot_w64(m != 0u);
      const int pos = cnt + (int)__builtin_amdgcn_mbcnt_hi((unsigned)(bal >> 32),
                                                           __builtin_amdgcn_mbcnt_lo((unsigned)bal, 0u));
      if (m != 0u) work[wave][pos] = make_uint2(m, (unsigned)(64 * q + lane));
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
  sig += __shfl_xor(sig, 32);
  sig = ibk != 0.0f ? sig * ibk : 0.0f;
  const int64_t kbase = ((int64_t)slab * RG + rg) * KP + (int64_t)kb * 32;
#pragma unroll
  for (int i = 0; i < 16; ++i) {
    float* dst = part_mu + (kbase + acc_row(i, g)) * DP + NJ * c;
#pragma unroll
    for (int jj = 0; jj < NJ; ++jj) dst[jj] = acc[jj][i];
  }
  if (g == 0) {
    part_nk[kbase + c] = nk;
    part_sig[kbase + c] = sig;
  }
}

// ---------------------------------------------------------------------------
// Finish: fixed-order fp64 reduction over slabs (deterministic).
// ---------------------------------------------------------------------------
__global__ __launch_bounds__(256) void iso_reduce(const float* __restrict__ part_mu,
                                                  const float* __restrict__ part_nk,
                                                  const float* __restrict__ part_sig, int nslab,
                                                  int KP, int DP, int64_t K, int D,
                                                  float* __restrict__ Nk, float* __restrict__ mu_acc,
                                                  float* __restrict__ sig_acc, int accumulate) {
  const int64_t idx = (int64_t)blockIdx.x * blockDim.x + threadIdx.x;
  const int W = D + 2;
  if (idx >= K * W) return;
  const int64_t k = idx / W;
  const int col = (int)(idx % W);
  double s = 0.0;
  if (col < D) {
    s = strided_sum(part_mu + k * DP + col, nslab, (int64_t)KP * DP);
    float* o = mu_acc + k * D + col;
    *o = accumulate ? (float)((double)*o + s) : (float)s;
  } else if (col == D) {
    s = strided_sum(part_nk + k, nslab, KP);
    Nk[k] = accumulate ? (float)((double)Nk[k] + s) : (float)s;
  } else {
    s = strided_sum(part_sig + k, nslab, KP);
    sig_acc[k] = accumulate ? (float)((double)sig_acc[k] + s) : (float)s;
  }
}

// The same finish with one wave per output element, for many partials (few
// components over many row slabs).
__global__ __launch_bounds__(256) void iso_reduce_wide(const float* __restrict__ part_mu,
                                                       const float* __restrict__ part_nk,
                                                       const float* __restrict__ part_sig, int nslab,
                                                       int KP, int DP, int64_t K, int D,
                                                       float* __restrict__ Nk, float* __restrict__ mu_acc,
                                                       float* __restrict__ sig_acc, int accumulate) {
  const int64_t idx = (int64_t)blockIdx.x * 4 + (threadIdx.x >> 6);
  const int lane = threadIdx.x & 63;
  const int W = D + 2;
  if (idx >= K * W) return;
  const int64_t k = idx / W;
  const int col = (int)(idx % W);
  if (col < D) {
    const double s = wave_strided_sum(part_mu + k * DP + col, nslab, (int64_t)KP * DP, lane);
    float* o = mu_acc + k * D + col;
    if (lane == 0) *o = accumulate ? (float)((double)*o + s) : (float)s;
  } else if (col == D) {
    const double s = wave_strided_sum(part_nk + k, nslab, KP, lane);
    if (lane == 0) Nk[k] = accumulate ? (float)((double)Nk[k] + s) : (float)s;
  } else {
    const double s = wave_strided_sum(part_sig + k, nslab, KP, lane);
    if (lane == 0) sig_acc[k] = accumulate ? (float)((double)sig_acc[k] + s) : (float)s;
  }
}

// Atomic finish: every slab partial is added into the (zeroed or accumulated) outputs.
__global__ __launch_bounds__(256) void iso_reduce_atomic(const float* __restrict__ part_mu,
                                                         const float* __restrict__ part_nk,
                                                         const float* __restrict__ part_sig, int nslab,
                                                         int KP, int DP, int64_t K, int D,
                                                         float* __restrict__ Nk, float* __restrict__ mu_acc,
                                                         float* __restrict__ sig_acc) {
  const int64_t idx = (int64_t)blockIdx.x * blockDim.x + threadIdx.x;
  const int W = D + 2;
  const int sl = blockIdx.y;
  if (idx >= K * W || sl >= nslab) return;
  const int64_t k = idx / W;
  const int col = (int)(idx % W);
  if (col < D)
    atomicAdd(mu_acc + k * D + col, part_mu[((int64_t)sl * KP + k) * DP + col]);
  else if (col == D)
    atomicAdd(Nk + k, part_nk[(int64_t)sl * KP + k]);
  else
    atomicAdd(sig_acc + k, part_sig[(int64_t)sl * KP + k]);
}

__global__ __launch_bounds__(256) void fill_f32(float* __restrict__ p, int64_t n, float v) {
  const int64_t i = (int64_t)blockIdx.x * blockDim.x + threadIdx.x;
  if (i < n) p[i] = v;
}

// Above D = 128: pass 1 is iso_lse_ctile for both plans; pass 2 of the default plan
// (any D) is iso_accum_drange, that of the stored plan (D <= 256) launch_passes'.
hipError_t launch_ctile(const IsoPlan& pl, const float* X, int64_t ldx, unsigned char* ws, float* logZ,
                        bool run1, bool run2, bool dense, hipStream_t stream) {
  const bf16x8* mu3 = reinterpret_cast<const bf16x8*>(ws + pl.off_mu3);
  double2* rowstat = reinterpret_cast<double2*>(ws + pl.off_rowstat);
  unsigned* ljmask = reinterpret_cast<unsigned*>(ws + pl.off_ljmask);
  unsigned* ljcount = reinterpret_cast<unsigned*>(ws + pl.off_ljcount);
  const int NQ = pl.DP / 16;
  if (run1 && !pl.lj && lse_in_regs(pl.DP)) {
    // D = 192, 256: the register-resident pass 1 (same operands, chains and order).
    auto lse = [&](auto dp_tag) -> hipError_t {
      constexpr int DP = decltype(dp_tag)::value;
      const size_t lds1 = lse_lds_base(DP) + (pl.rexact ? (size_t)kWaves * 32 * pl.KB * 2 : 0);
      hipError_t e = hipFuncSetAttribute(reinterpret_cast<const void*>(&iso_lse<DP, kLjmNeed>),
                                         hipFuncAttributeMaxDynamicSharedMemorySize, (int)lds1);
      if (e != hipSuccess) return e;
      hipLaunchKernelGGL((iso_lse<DP, kLjmNeed>), dim3((unsigned)cdiv(pl.N, 32 * kWaves)), dim3(kThreads), lds1,
                         stream, X, ldx, pl.N, (int)pl.D, mu3, reinterpret_cast<const double2*>(ws + pl.off_kcblk),
                         pl.KB, logZ, rowstat, nullptr, nullptr, ljmask, ljcount, dense ? 1 : 0,
                         pl.rexact ? 1 : 0);
      return hipGetLastError();
    };
    hipError_t e = pl.DP == 192 ? lse(std::integral_constant<int, 192>{}) : lse(std::integral_constant<int, 256>{});
    if (e != hipSuccess) return e;
  } else if (run1) {
    const bool exact = pl.rexact && !pl.lj;
    const int ctb = ctile_blocks(pl.DP);
    const size_t lds1 = lse_ctile_base(ctb) + (exact ? (size_t)kCtWaves * 32 * pl.KB * 2 : 0);
    auto kern = pl.lj ? (ctb == 2 ? &iso_lse_ctile<kLjmStore, 2> : &iso_lse_ctile<kLjmStore, 4>)
                      : (ctb == 2 ? &iso_lse_ctile<kLjmNeed, 2> : &iso_lse_ctile<kLjmNeed, 4>);
    hipError_t e = hipFuncSetAttribute(reinterpret_cast<const void*>(kern),
                                       hipFuncAttributeMaxDynamicSharedMemorySize, (int)lds1);
    if (e != hipSuccess) return e;
    hipLaunchKernelGGL(kern, dim3((unsigned)cdiv(pl.N, 32 * kCtWaves)), dim3(64 * kCtWaves), lds1,
                       stream, X, ldx, pl.N, (int)pl.D, NQ, mu3,
                       reinterpret_cast<const double2*>(ws + pl.off_kcblk), pl.KB, logZ, rowstat,
                       pl.lj ? reinterpret_cast<float*>(ws + pl.off_lj) : nullptr,
                       pl.lj ? reinterpret_cast<float*>(ws + pl.off_ljmax) : nullptr, ljmask, ljcount,
                       dense ? 1 : 0, exact ? 1 : 0);
  }
  if (run2 && !pl.lj) {
    const size_t lds2 = accum_drange_lds_bytes(pl.DP < kDrange ? pl.DP : kDrange);
    hipError_t e = hipFuncSetAttribute(reinterpret_cast<const void*>(&iso_accum_drange),
                                       hipFuncAttributeMaxDynamicSharedMemorySize, (int)lds2);
    if (e != hipSuccess) return e;
    const int64_t items = (int64_t)pl.KB * pl.nslab * pl.ndr;
    hipLaunchKernelGGL(iso_accum_drange, dim3((unsigned)(8 * cdiv(items, 8))), dim3(64 * kCtWaves), lds2,
                       stream, X, ldx, pl.N, (int)pl.D, NQ, pl.DP, mu3,
                       reinterpret_cast<const double4*>(ws + pl.off_kcgat), pl.KB, pl.KP, rowstat, ljmask,
                       pl.nslab, pl.rows_per_slab, pl.ndr, reinterpret_cast<float*>(ws + pl.off_part_mu),
                       reinterpret_cast<float*>(ws + pl.off_part_nk),
                       reinterpret_cast<float*>(ws + pl.off_part_sig), dense ? 1 : 0);
  }
  return hipGetLastError();
}

// The default plan up to D = 128, the stored plan's passes up to D = 128 and its
// pass 2 above (pass 1 there is launch_ctile's).
template <int DP>
hipError_t launch_passes(const IsoPlan& pl, const float* X, int64_t ldx, unsigned char* ws,
                         float* logZ, bool run1, bool run2, bool dense, hipStream_t stream) {
  const double2* kc_blk = reinterpret_cast<const double2*>(ws + pl.off_kcblk);
  const double4* kc_lin = reinterpret_cast<const double4*>(ws + pl.off_kclin);
  double2* rowstat = reinterpret_cast<double2*>(ws + pl.off_rowstat);
  float* pmu = reinterpret_cast<float*>(ws + pl.off_part_mu);
  float* pnk = reinterpret_cast<float*>(ws + pl.off_part_nk);
  float* psig = reinterpret_cast<float*>(ws + pl.off_part_sig);
  float* lj = (pl.lj || pl.autolj) ? reinterpret_cast<float*>(ws + pl.off_lj) : nullptr;
  unsigned* ljmask = reinterpret_cast<unsigned*>(ws + pl.off_ljmask);
  unsigned* ljcount = reinterpret_cast<unsigned*>(ws + pl.off_ljcount);
  if (run1) {
    if constexpr (DP <= 128) {
      hipError_t e = hipSuccess;
      if (pl.need || pl.lj) {
        // The software-pipelined pass 1 (the stored plan's also writes the log-joint;
        // with FGMM_FLAG_STORE_LOGJOINT_AUTO the probe's selector decides first).
        unsigned* probe = pl.autolj ? reinterpret_cast<unsigned*>(ws + pl.off_probe) : nullptr;
        if (pl.autolj)
          hipLaunchKernelGGL((iso_store_probe<DP>), dim3((unsigned)pl.nprobe), dim3(64 * kProbeWaves), 0, stream, X, ldx, pl.N,
                             (int)pl.D, reinterpret_cast<const bf16x8*>(ws + pl.off_mu3), kc_blk, pl.KB, pl.nprobe,
                             probe);
        const ProbeSel psel = probe ? ProbeSel{probe, pl.nprobe, probe_min_pairs(pl.N, pl.nprobe, pl.KB)}
                                    : ProbeSel{nullptr, 0, 0};
        const bool st = pl.lj || pl.autolj;
        const size_t lds1 = lse_pipe_lds_bytes<DP>() + (pl.rexact ? (size_t)kPipeWaves * 32 * pl.KB * 2 : 0) +
                            (st ? kPipeStoreLds : 0);
        auto kern = pl.rexact ? &iso_lse_pipe<DP, 1> : &iso_lse_pipe<DP, 0>;
        if (lds1 > 65536)
          e = hipFuncSetAttribute(reinterpret_cast<const void*>(kern), hipFuncAttributeMaxDynamicSharedMemorySize,
                                  (int)lds1);
        if (e != hipSuccess) return e;
        const PipeGrid pg = pipe_grid(pl.N);
        hipLaunchKernelGGL(kern, dim3((unsigned)pg.grid), dim3(kPipeThreads), lds1, stream,
                           X, ldx, pl.N, (int)pl.D, reinterpret_cast<const bf16x8*>(ws + pl.off_mu3), kc_blk,
                           pl.KB, logZ, rowstat, ljmask, ljcount, dense ? 1 : 0, lj, psel,
                           reinterpret_cast<__bf16*>(ws + pl.off_xsplit), reinterpret_cast<float2*>(ws + pl.off_zpair),
                           pg.full, pg.small);
      }
    } else {
      return hipErrorInvalidValue;   // launch_ctile runs pass 1 above D = 128
    }
  }
  if (!run2) return hipGetLastError();
  if constexpr (DP <= 128) {
    if (pl.need) {
      // Both forms are launched; the needed-row count pass 1 left selects one on the
      // device: the gathering kernel below three quarters of all (row, block) pairs
      // (measured at N=1M K=1024: at a quarter it takes half the tile kernel's time, with
      // every pair needed 1.1-1.25 times it).
      const int64_t dense_min = cdiv(cdiv(pl.N, 32) * 32 * (int64_t)pl.KB * 3, 4);
      // FGMM_FLAG_STORE_LOGJOINT_AUTO: the stored branch (iso_accum_ljt over the same
      // slabs and partials) is launched too; the probe's selector picks one side.
      const ProbeSel sel = pl.autolj ? ProbeSel{reinterpret_cast<const unsigned*>(ws + pl.off_probe), pl.nprobe,
                                                probe_min_pairs(pl.N, pl.nprobe, pl.KB)}
                                     : ProbeSel{nullptr, 0, 0};
      if (pl.autolj) {
        constexpr size_t ldsj = LjtShape<DP>::lds;
        static_assert(ldsj <= kMaxLds, "stored pass-2 stages exceed LDS");
        hipError_t ej = hipFuncSetAttribute(reinterpret_cast<const void*>(&iso_accum_ljt<DP>),
                                            hipFuncAttributeMaxDynamicSharedMemorySize, (int)ldsj);
        if (ej != hipSuccess) return ej;
        const int ncg = (int)cdiv(pl.KB, kLjtWaves);
        hipLaunchKernelGGL((iso_accum_ljt<DP>), dim3((unsigned)ljt_grid(pl.nslab, ncg)), dim3(64 * kLjtWaves), ldsj,
                           stream, lj, reinterpret_cast<const __bf16*>(ws + pl.off_xsplit),
                           reinterpret_cast<const float2*>(ws + pl.off_zpair), pl.N, ljmask, ljcount, (int64_t)-1,
                           sel, kc_lin, pl.KB, pl.KP, pl.nslab, pl.rows_per_slab, ncg, pmu, pnk, psig,
                           dense ? 1 : 0);
      }
      constexpr size_t lds = gather_lds_bytes(DP);
      static_assert(lds <= kMaxLds, "gathering pass 2 exceeds LDS");
      hipError_t e = hipFuncSetAttribute(reinterpret_cast<const void*>(&iso_accum_gather<DP>),
                                         hipFuncAttributeMaxDynamicSharedMemorySize, (int)lds);
      if (e != hipSuccess) return e;
      // Above D = 64 the gather runs one wave per SIMD: where its (slab, block) items
      // would take two rounds of waves, each wave takes two slabs in turn (C2, same
      // box: 0.221 -> 0.197 ms), keeping the slabs and partials the stored branch's
      // pass 2 shares.
      const int spw = (DP > 64 && (int64_t)pl.nslab * pl.KB >= (int64_t)2 * 4 * current_device_cus()) ? 2 : 1;
      hipLaunchKernelGGL(iso_accum_gather<DP>, dim3((unsigned)gather_grid(pl.nslab, pl.KB, spw)),
                         dim3(64 * kGatherWaves), lds, stream, X, ldx, pl.N, (int)pl.D,
                         reinterpret_cast<const bf16x8*>(ws + pl.off_mu3),
                         reinterpret_cast<const double4*>(ws + pl.off_kcgat), pl.KB, pl.KP, rowstat,
                         ljmask, ljcount, dense_min, pl.nslab, pl.rows_per_slab, pmu, pnk, psig,
                         dense ? 1 : 0, sel, spw);
      // The tile pass: one wave per block up to D = 64, a pair of waves (one chain
      // each) at D = 96 and 128.
      auto tiles = [&](auto kern, size_t lds_t, int waves) -> hipError_t {
        hipError_t et = hipFuncSetAttribute(reinterpret_cast<const void*>(kern),
                                            hipFuncAttributeMaxDynamicSharedMemorySize, (int)lds_t);
        if (et != hipSuccess) return et;
        hipLaunchKernelGGL(kern, dim3((unsigned)(pl.nslab * cdiv(pl.KB, kTileBlocks))), dim3(64 * waves), lds_t,
                           stream, X, ldx, pl.N, (int)pl.D, reinterpret_cast<const bf16x8*>(ws + pl.off_mu3),
                           reinterpret_cast<const double4*>(ws + pl.off_kcgat), pl.KB, pl.KP, rowstat, ljmask,
                           ljcount, dense_min, pl.nslab, pl.rows_per_slab, pmu, pnk, psig, dense ? 1 : 0, sel);
        return hipGetLastError();
      };
      if constexpr (DP > 64) {
        static_assert(tiles2_lds_bytes(DP) <= kMaxLds, "tile pass 2 exceeds LDS");
        return tiles(&iso_accum_tiles2<DP>, tiles2_lds_bytes(DP), kTileWaves2);
      } else {
        static_assert(tiles_lds_bytes(DP) <= kMaxLds, "tile pass 2 exceeds LDS");
        return tiles(&iso_accum_tiles<DP>, tiles_lds_bytes(DP), kTileBlocks);
      }
    }
  }
  if (!pl.lj) return hipErrorInvalidValue;   // not a plan of this launcher
  if constexpr (DP <= 128) {
    // Sparse masks (on average at most 3 needed rows per tile and block) go to
    // iso_accum_sparse where it applies (D a multiple of 32, 64 to 128); both kernels
    // are launched and each returns unless the needed-row count selects it.
    int64_t sparse_max = -1;
    if constexpr (DP >= 64) {
      if (pl.D == DP) {
        sparse_max = 3 * cdiv(pl.N, 32) * pl.KB;
        const int64_t nw = (int64_t)pl.nslab * pl.rgroups * pl.KB;
        hipLaunchKernelGGL((iso_accum_sparse<DP>), dim3((unsigned)cdiv(nw, kSparseWaves)),
                           dim3(64 * kSparseWaves), 0, stream, X, ldx, pl.N, lj, ljmask, ljcount,
                           sparse_max, kc_lin, pl.KB, pl.KP, rowstat, pl.nslab, pl.rgroups,
                           pl.rows_per_slab, pmu, pnk, psig, dense ? 1 : 0);
      }
    }
    constexpr size_t lds = LjtShape<DP>::lds;
    static_assert(lds <= kMaxLds, "stored pass-2 stages exceed LDS");
    hipError_t el = hipFuncSetAttribute(reinterpret_cast<const void*>(&iso_accum_ljt<DP>),
                                        hipFuncAttributeMaxDynamicSharedMemorySize, (int)lds);
    if (el != hipSuccess) return el;
    hipLaunchKernelGGL((iso_accum_ljt<DP>), dim3((unsigned)ljt_grid(pl.nslab, pl.ncg)), dim3(64 * kLjtWaves), lds,
                       stream, lj, reinterpret_cast<const __bf16*>(ws + pl.off_xsplit),
                       reinterpret_cast<const float2*>(ws + pl.off_zpair), pl.N, ljmask, ljcount, sparse_max,
                       ProbeSel{nullptr, 0, 0}, kc_lin, pl.KB, pl.KP, pl.nslab, pl.rows_per_slab, pl.ncg, pmu, pnk,
                       psig, dense ? 1 : 0);
    return hipGetLastError();
  }
  const dim3 grid2((unsigned)(pl.nslab * pl.ncg));
  const int64_t sparse_max = -1;
  auto launch = [&](auto cb_tag, auto nh_tag) -> hipError_t {
    constexpr int CB = decltype(cb_tag)::value;
    constexpr int NH = decltype(nh_tag)::value;
    constexpr size_t lds = accum_lj_lds_bytes<DP, CB, NH>();
    static_assert(lds <= kMaxLds, "pass-2 tiles exceed LDS");
    if (lds > 65536) {
      hipError_t e = hipFuncSetAttribute(reinterpret_cast<const void*>(&iso_accum_lj<DP, CB, NH>),
                                         hipFuncAttributeMaxDynamicSharedMemorySize, (int)lds);
      if (e != hipSuccess) return e;
    }
    hipLaunchKernelGGL((iso_accum_lj<DP, CB, NH>), grid2, dim3(kAccThreads), lds, stream, X, ldx,
                       pl.N, (int)pl.D, lj, ljmask, ljcount, sparse_max, kc_lin, pl.KB, pl.KP,
                       rowstat, pl.nslab,
                       pl.rows_per_slab, pmu, pnk, psig, dense ? 1 : 0);
    return hipSuccess;
  };
  using I1 = std::integral_constant<int, 1>;
  using I4 = std::integral_constant<int, 4>;
  hipError_t e = hipSuccess;
  if constexpr (DP > 128) {
    if (DP <= 192 && pl.cpg == 8) {
      if constexpr (DP <= 192) e = launch(std::integral_constant<int, 8>{}, I1{});
    } else {
      e = launch(I4{}, std::integral_constant<int, 2>{});
    }
  }
  if (e != hipSuccess) return e;
  return hipGetLastError();
}

// ===========================================================================
// bf16 operand contract (FGMM_FLAG_BF16), the arithmetic of the reference's H100
// kernels (flash_gmm_h100.py:247-328): X and mu rounded to bfloat16 for x.mu and for
// r^T X (r rounded to bfloat16 there), fp32 accumulation, constants from the fp32
// mu, everything else in fp32 log2 units:
//   ish_k = 0.5 exp(-lss_k) log2 e,  c0_k = (lpi_k - 0.5 D (log 2pi + lss_k)) log2 e - ish_k ||mu_k||^2
//   ll2 = c0_k - ish_k ||x_b||^2 + 2 ish_k (x_b . mu_b)
// The matrix step is v_mfma_f32_32x32x16_bf16: 16 dimensions (or rows) per step;
// the hardware pairs element e of lane-half g of A with the same (g, e) of B, so
// both operands take dimensions 16q + 8g + e.  Pass 2 recomputes the contraction
// (at bf16 rates that costs less than storing the log-joint).
// ===========================================================================
// Above D = 128 pass 2 splits a component block over two waves, one half of the
// dimensions each (and pass 1 sums its contraction in the same two halves).
__host__ __device__ constexpr int bf16_halves(int DP) { return DP > 128 ? 2 : 1; }

// Prologue: mu in operand order mu_op[kb][q][lane] = mu[kb*32 + lane%32][16q + 8(lane/32) + e]
// (bf16x8), and per component {c0, ish, 2 ish, ||mu||^2} in fp32 (formed in fp64).
__global__ __launch_bounds__(64) void iso_bf16_prep(const float* __restrict__ mu, int64_t ldmu,
                                                    int64_t K, int D, int DP,
                                                    const float* __restrict__ lss,
                                                    const float* __restrict__ lpi,
                                                    bf16x8* __restrict__ mu_op, f32x4* __restrict__ kc,
                                                    unsigned* __restrict__ ljcount) {
  const int kb = blockIdx.x, lane = threadIdx.x, c = lane & 31, g = lane >> 5;
  if (ljcount && kb == 0) ljcount[lane] = 0u;   // pass 1 counts the needed pairs into these
  const int64_t k = (int64_t)kb * 32 + c;
  const bool valid = k < K;
  const int NC = DP / 16;
  for (int q = 0; q < NC; ++q) {
    bf16x8 v;
#pragma unroll
    for (int e = 0; e < 8; ++e) {
      const int d = 16 * q + 8 * g + e;
      v[e] = (__bf16)((valid && d < D) ? mu[k * ldmu + d] : 0.0f);
    }
    mu_op[((int64_t)kb * NC + q) * 64 + lane] = v;
  }
  if (g == 0) {
    f32x4 w = {-INFINITY, 0.0f, 0.0f, 0.0f};
    if (valid) {
      double msq = 0.0;
      for (int d = 0; d < D; ++d) {
        const double m = (double)mu[k * ldmu + d];
        msq = fma(m, m, msq);
      }
      const double l = (double)lss[k];
      const double ish = 0.5 * exp(-l) * kLog2e;
      const double c0 = ((double)lpi[k] - 0.5 * (double)D * (kLog2Pi + l)) * kLog2e - ish * msq;
      w = f32x4{(float)c0, (float)ish, (float)(2.0 * ish), (float)msq};
    }
    kc[k] = w;
  }
}

// Pass 1: grid over 128-row tiles, 4 waves of 32 rows.  X is rounded to bf16 in
// registers as it is loaded; mu blocks (bf16 operands + constants) stream through an
// LDS double buffer.  Writes logZ and per-row {logZ2, ||x_b||^2} (fp32).  With NEED
// each row's block maximum, rounded up to bf16, stays in LDS, and once logZ2 is final
// the need words (bit r of (tile, block) set unless row r's maximum lies kLjNeedGap
// below its logZ2, so that every responsibility of a cleared pair is exactly zero in
// fp32) and the needed-pair count are written, as the fp32 default plan does.
template <int DP>
constexpr size_t bf16_lse_lds_bytes() {
  static_assert(bf16_lse_lds_base(DP) == (size_t)2 * (DP / 16) * 64 * sizeof(bf16x8) + (size_t)2 * 32 * sizeof(f32x4),
                "host sizing");
  return bf16_lse_lds_base(DP);
}

template <int DP, bool NEED = false>
__global__ __launch_bounds__(kThreads) void iso_bf16_lse(const float* __restrict__ X, int64_t ldx,
                                                         int64_t N, int D,
                                                         const bf16x8* __restrict__ mu_op,
                                                         const f32x4* __restrict__ kc, int KB,
                                                         float* __restrict__ logZ,
                                                         float2* __restrict__ rowstat,
                                                         unsigned* __restrict__ ljmask,
                                                         unsigned* __restrict__ ljcount, int dense) {
  constexpr int NC = DP / 16;
  constexpr int BLK = NC * 64;                 // bf16x8 per 32-component block
  constexpr int LPT = (BLK + kThreads - 1) / kThreads;

  extern __shared__ __align__(16) unsigned char lds_raw[];
  bf16x8* mu_l = reinterpret_cast<bf16x8*>(lds_raw);                                // [2][BLK]
  f32x4* kc_l = reinterpret_cast<f32x4*>(lds_raw + 2 * BLK * sizeof(bf16x8));      // [2][32]
  unsigned short* rmax_l = reinterpret_cast<unsigned short*>(lds_raw + bf16_lse_lds_bytes<DP>());   // [wave][KB][32]

  const int tid = threadIdx.x, lane = tid & 63, wave = tid >> 6;
  const int c = lane & 31, g = lane >> 5;
  const int64_t tile = (int64_t)blockIdx.x * kWaves + wave;
  const int64_t row = tile * 32 + c;
  const bool valid = row < N;

  bf16x8 st[LPT];
  f32x4 kst = {0.0f, 0.0f, 0.0f, 0.0f};
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

  // This lane's operand chunks: row `row`, dimensions 16q + 8g .. +7, rounded to bf16.
  bf16x8 xb[NC];
  float xsq = 0.0f;
#pragma unroll
  for (int q = 0; q < NC; ++q) {
    const int d0 = 16 * q + 8 * g;
    xb[q] = to_bf16x8(load_row4(X, ldx, row, d0, D, valid), load_row4(X, ldx, row, d0 + 4, D, valid));
#pragma unroll
    for (int e = 0; e < 8; ++e) {
      const float v = (float)xb[q][e];
      xsq = fmaf(v, v, xsq);
    }
  }
  xsq += __shfl_xor(xsq, 32);
  commit(0);
  lds_barrier();

  float mx = -INFINITY, sm = 0.0f;
  for (int kb = 0; kb < KB; ++kb) {
    const int buf = kb & 1;
    const bool more = kb + 1 < KB;
    if (more) fetch(kb + 1);
    const bf16x8* mp = mu_l + buf * BLK + lane;
    // S^T = mu . X^T: lane = row, register i = component acc_row(i, g).  Above D = 128
    // the two halves of D run as separate chains added at the end, the order pass 2
    // uses, so both passes form bitwise the same log-joint.
    f32x16 acc = zero16();
    if constexpr (bf16_halves(DP) == 2) {
      f32x16 acc1 = zero16();
#pragma unroll
      for (int q = 0; q < NC / 2; ++q) {
        acc = mfma_bf16(mp[q * 64], xb[q], acc);
        acc1 = mfma_bf16(mp[(q + NC / 2) * 64], xb[q + NC / 2], acc1);
      }
#pragma unroll
      for (int i = 0; i < 16; ++i) acc[i] += acc1[i];
    } else {
#pragma unroll
      for (int q = 0; q < NC; ++q) acc = mfma_bf16(mp[q * 64], xb[q], acc);
    }
    const f32x4* kp = kc_l + buf * 32;
    float ll[16];
    float bm = -INFINITY;
#pragma unroll
    for (int i = 0; i < 16; ++i) {
      const f32x4 w = kp[acc_row(i, g)];
      ll[i] = fmaf(w.z, acc[i], fmaf(-w.y, xsq, w.x));
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
    rowstat[row] = make_float2(lz2, xsq);
    if (logZ) logZ[row] = lz2 * (float)kLn2;
  }
  if constexpr (NEED) {
    // Pass 2 forms fl(ll2 - logZ2) with ll2 <= the bound, so a cleared pair gives
    // 2^x = 0 there (lz2 is a float: need_put_masks' low part is 0).
    const unsigned short* rm = rmax_l + wave * KB * 32 + c;
    if (g == 0)
      need_put_masks([&](int kb) { return bf16_bits_to_float(rm[kb * 32]); }, ljmask + tile * KB,
                     ljcount + (tile & 63), KB, c, (double)lz2, valid, dense != 0);
  }
}

// Pass 2: grid over (row slab x group of CB component blocks); 8 waves = CB blocks x
// NH halves of the dimensions x 8/(CB NH) row groups.  With NH = 2 each wave forms the
// partial S over its half, the halves meet in LDS and are added in a fixed order (both
// waves then hold the same r), and each accumulates r^T X for its half of the columns.
// X super-tiles are loaded coalesced (consecutive lanes, consecutive 16 bytes of a
// row), rounded to bf16 once per workgroup and held row-major in LDS: the A operand of
// the recomputed S = X mu^T is a 16-byte read per lane, and the B operand of r^T X (8
// consecutive rows of one column per lane-half) comes from two transposing reads
// (lds_rows_operand).  r leaves S in the accumulator layout (lane = component,
// register = row 8q + 4g + j); one v_permlane32_swap per register pair gives each
// half-wave 8 consecutive rows, the A-operand layout of r^T X, with no trip through LDS.
// The row stride (DP + 16 bf16) is an odd multiple of 32 bytes, the stride the
// transposing reads want.
__host__ __device__ constexpr int bf16_xr_stride(int DP) { return DP + 16; }   // bf16 per X row
// The next super-tile waits in registers (float4 per thread) while this one is
// processed: at most 8 float4 where the halves of D need no exchange, 6 where they do
// (its buffer and the two halves' sums take the rest); more spills to scratch.
__host__ __device__ constexpr int bf16_stage_cap(int DP) { return bf16_halves(DP) == 1 ? 8 : 6; }
__host__ __device__ constexpr int bf16_stage_f4(int TR, int DP) { return TR * (DP / 4) / kAccThreads; }
// Row groups each wave takes per super-tile: two where the halves of D need no
// exchange, so every barrier and every tile load covers twice the work.
__host__ __device__ constexpr int bf16_rows_per_wave(int DP) { return bf16_halves(DP) == 1 ? 2 : 1; }
__host__ __device__ constexpr int bf16_tile_rows(int DP, int CB) {
  return 32 * (kAccWaves / (CB * bf16_halves(DP))) * bf16_rows_per_wave(DP);
}
__host__ __device__ constexpr size_t bf16_accum_lds_bytes(int DP, int CB) {
  return (size_t)2 * ((size_t)bf16_tile_rows(DP, CB) * bf16_xr_stride(DP)) * 2 +
         (size_t)2 * bf16_tile_rows(DP, CB) * sizeof(float2) +
         (bf16_halves(DP) > 1 ? (size_t)kAccWaves * 16 * 64 * sizeof(float) : 0);
}
// Whether iso_bf16_accum<DP, CB> fits: its tiles in LDS, its staging within the cap.
__host__ __device__ constexpr bool bf16_accum_fits(int DP, int CB) {
  return bf16_accum_lds_bytes(DP, CB) <= kMaxLds &&
         bf16_stage_f4(bf16_tile_rows(DP, CB), DP) <= bf16_stage_cap(DP);
}
// Component blocks per workgroup: as few as K has (no idle waves), unless that shape
// does not fit; 4 always does.
__host__ inline int bf16_blocks_per_group(int DP, int KB) {
  if (KB <= 1 && bf16_accum_fits(DP, 1)) return 1;
  if (KB <= 2 && bf16_accum_fits(DP, 2)) return 2;
  return 4;
}

template <int DP, int CB, int NH = bf16_halves(DP)>
__global__ __attribute__((amdgpu_flat_work_group_size(kAccThreads, kAccThreads), amdgpu_waves_per_eu(2, 2)))
void iso_bf16_accum(const float* __restrict__ X, int64_t ldx, int64_t N, int D,
                    const bf16x8* __restrict__ mu_op, const f32x4* __restrict__ kc, int KB, int KP,
                    const float2* __restrict__ rowstat, int nslab, int64_t rows_per_slab,
                    float* __restrict__ part_mu, float* __restrict__ part_nk,
                    float* __restrict__ part_sig, int dense, const unsigned* __restrict__ needcount,
                    int64_t dense_min) {
  constexpr int NC = DP / 16 / NH;             // 16-dimension chunks of the contraction per wave
  constexpr int NJ = DP / 32 / NH;             // 32-column tiles of r^T X per wave
  constexpr int RG = kAccWaves / (CB * NH);    // row groups of waves (32 rows each)
  constexpr int RPW = bf16_rows_per_wave(DP);  // row groups per wave per super-tile
  constexpr int TR = bf16_tile_rows(DP, CB);   // rows per super-tile, 32 RG RPW
  constexpr int XR = bf16_xr_stride(DP);
  constexpr int V4 = DP / 4;
  constexpr int NV = TR * V4;                  // float4 per super-tile
  constexpr int LPT = (NV + kAccThreads - 1) / kAccThreads;
  static_assert(kAccWaves % (CB * NH) == 0 && NV % kAccThreads == 0 && (DP / 32) % NH == 0,
                "even split");

  // With need masks and fewer than dense_min needed pairs iso_bf16_gather runs instead
  // (uniform exit).
  if (needcount && need_total(needcount) < dense_min) return;

  extern __shared__ __align__(16) unsigned char lds_raw[];
  __bf16* xr = reinterpret_cast<__bf16*>(lds_raw);                        // [2][TR][XR]
  float2* rs = reinterpret_cast<float2*>(xr + 2 * TR * XR);                // [2][TR]
  float* ex = reinterpret_cast<float*>(rs + 2 * TR);                       // [8][16][64] (NH = 2)

  const int tid = threadIdx.x, lane = tid & 63, wave = tid >> 6;
  const int c = lane & 31, g = lane >> 5;
  const int cbw = wave % CB, h = (wave / CB) % NH, rg = wave / (CB * NH);
  const int d0 = h * (DP / NH);                // first dimension of this wave's half
  const int slab = blockIdx.x % nslab;
  const int cg = blockIdx.x / nslab;
  const int kb = cg * CB + cbw;
  const bool active = kb < KB;

  const int64_t r_begin = (int64_t)slab * rows_per_slab;
  int64_t r_end = r_begin + rows_per_slab;
  if (r_end > N) r_end = N;
  const int ntiles = r_end > r_begin ? (int)cdiv(r_end - r_begin, TR) : 0;

  // B operand of the recompute (lane = component, dimensions 16q + 8g + e) and the
  // component's constants.
  bf16x8 mub[NC];
  f32x4 w = {-INFINITY, 0.0f, 0.0f, 0.0f};
#pragma unroll
  for (int q = 0; q < NC; ++q) {
    if (active) {
      mub[q] = mu_op[((int64_t)kb * (NC * NH) + h * NC + q) * 64 + lane];
    } else {
#pragma unroll
      for (int e = 0; e < 8; ++e) mub[q][e] = (__bf16)0.0f;
    }
  }
  if (active) w = kc[(int64_t)kb * 32 + c];
  const float ish = w.y, ish2 = w.z, musq = w.w, c0 = w.x;

  f32x16 acc[NJ];
#pragma unroll
  for (int j = 0; j < NJ; ++j) acc[j] = zero16();
  // sig = sum r (||x||^2 - 2 x.mu + ||mu||^2) = srx - 2 srs + ||mu||^2 nk, from two running sums.
  float nk = 0.0f, srx = 0.0f, srs = 0.0f;

  // X super-tiles go global -> registers -> LDS (double-buffered): tile t + 1 is
  // loaded while tile t is processed.
  f32x4 stage[LPT];
  float2 rstage = make_float2(INFINITY, 0.0f);
  const bool full_d = (D == DP);
  // float4 idx of a super-tile <-> (row, 4 dimensions), row-major.
  auto tile_row = [](int idx) { return idx / V4; };
  auto tile_col = [](int idx) { return (idx % V4) * 4; };
  auto fetch = [&](int t, f32x4 (&stage)[LPT], float2& rstage) {
    const int64_t row0 = r_begin + (int64_t)t * TR;
    if (full_d && row0 + TR <= r_end) {
      const float* src = X + row0 * ldx;
#pragma unroll
      for (int q = 0; q < LPT; ++q) {
        const int idx = q * kAccThreads + tid;
        stage[q] = *reinterpret_cast<const f32x4*>(src + (int64_t)tile_row(idx) * ldx + tile_col(idx));
      }
    } else {
#pragma unroll
      for (int q = 0; q < LPT; ++q) {
        const int idx = q * kAccThreads + tid;
        const int64_t row = row0 + tile_row(idx);
        stage[q] = load_row4(X, ldx, row, tile_col(idx), D, row < r_end);
      }
    }
    if (tid < TR) {
      const int64_t row = row0 + tid;
      // Rows past the slab get logZ2 = +inf, hence r = 0.
      rstage = (row < r_end) ? rowstat[row] : make_float2(INFINITY, 0.0f);
    }
  };
  auto commit = [&](int buf, const f32x4 (&stage)[LPT], float2 rstage) {
    __bf16* dr = xr + buf * TR * XR;
#pragma unroll
    for (int q = 0; q < LPT; ++q) {
      const int idx = q * kAccThreads + tid;
      const f32x4 v = stage[q];
      typedef __bf16 bf16x4 __attribute__((ext_vector_type(4)));
      const bf16x4 b = {(__bf16)v.x, (__bf16)v.y, (__bf16)v.z, (__bf16)v.w};
      *reinterpret_cast<bf16x4*>(dr + tile_row(idx) * XR + tile_col(idx)) = b;
    }
    if (tid < TR) rs[buf * TR + tid] = rstage;
  };

  if (ntiles > 0) {
    fetch(0, stage, rstage);
    commit(0, stage, rstage);
  }
  lds_barrier();

  for (int t = 0; t < ntiles; ++t) {
    const int buf = t & 1;
    const bool more = t + 1 < ntiles;
    if (more) fetch(t + 1, stage, rstage);
#pragma unroll 1
    for (int u = 0; u < RPW; ++u) {
      const int rgu = u * RG + rg;                 // the wave's row group in this super-tile
      f32x16 s = zero16();
      if (active) {
        const __bf16* xrow = xr + buf * TR * XR + (rgu * 32 + c) * XR + d0 + 8 * g;
        // S = X mu^T for the wave's 32 rows: lane = component, register i = row acc_row(i, g).
#pragma unroll
        for (int q = 0; q < NC; ++q)
          s = mfma_bf16(*reinterpret_cast<const bf16x8*>(xrow + 16 * q), mub[q], s);
      }
      if constexpr (NH == 2) {
        // Add the two halves' partial S in a fixed order (half 0 + half 1).
        float* mine = ex + wave * 16 * 64 + lane;
#pragma unroll
        for (int i = 0; i < 16; ++i) mine[i * 64] = s[i];
        lds_barrier();
        const float* s0 = ex + (rg * CB * NH + cbw) * 16 * 64 + lane;
        const float* s1 = s0 + CB * 16 * 64;
#pragma unroll
        for (int i = 0; i < 16; ++i) s[i] = s0[i * 64] + s1[i * 64];
      }
      if (active) {
        const float2* rt = rs + buf * TR + rgu * 32;
        float r[16];
#pragma unroll
        for (int i = 0; i < 16; ++i) {
          const float2 z = rt[acc_row(i, g)];                 // {logZ2, ||x_b||^2}
          const float ll = fmaf(ish2, s[i], fmaf(-ish, z.y, c0));
          const float rv = fast_exp2(ll - z.x);
          if (h == 0) {
            nk += rv;
            srx = fmaf(rv, z.y, srx);
            srs = fmaf(rv, s[i], srs);
          }
          r[i] = rv;
        }
        bf16x8 a[2];
        acc_to_row_operands(r, a);
        // B operand: rows rgu*32 + 16p + 8g + e of column d0 + 32j + c.
        const __bf16* xt = xr + buf * TR * XR;
#pragma unroll
        for (int p = 0; p < 2; ++p) {
          // A step whose 16 rows x 32 components of bf16(r) are all zero adds nothing.
          if (dense || any_nonzero(a[p])) {
#pragma unroll
            for (int j = 0; j < NJ; ++j)
              acc[j] = mfma_bf16(a[p], lds_rows_operand(xt, XR, rgu * 32 + 16 * p, d0 + 32 * j, lane), acc[j]);
          }
        }
      }
    }
    if (more) commit(buf ^ 1, stage, rstage);
    lds_barrier();
  }

  if (active) {
    nk += __shfl_xor(nk, 32);
    srx += __shfl_xor(srx, 32);
    srs += __shfl_xor(srs, 32);
    const float sig = fmaf(musq, nk, fmaf(-2.0f, srs, srx));
    const int64_t kbase = ((int64_t)slab * RG + rg) * KP + (int64_t)kb * 32;
#pragma unroll
    for (int j = 0; j < NJ; ++j) {
#pragma unroll
      for (int i = 0; i < 16; ++i)
        part_mu[(kbase + acc_row(i, g)) * DP + d0 + 32 * j + c] = acc[j][i];
    }
    if (g == 0 && h == 0) {
      part_nk[kbase + c] = nk;
      part_sig[kbase + c] = sig;
    }
  }
}

// Pass 2 of the bf16 contract up to D = 128 where few pairs are needed (pass 1's
// needed-pair count below dense_min; iso_bf16_accum runs otherwise): one wave per
// (row slab, component block), 4 waves of one block on consecutive slabs per
// workgroup, the block's bf16 operands in LDS.  Each wave queues the rows whose need
// bit is set (queue_fill, as the fp32 gathering pass does) and per 32 queued rows:
//   - loads them (buffer resource over the slab: a lane without a row reads zeros),
//     rounds them to bf16 in the A-operand layout (lane = row) and writes them
//     row-major to its LDS tile;
//   - S = x_b . mu_b in the contraction order of pass 1 (one chain; the per-half sums
//     do not depend on the operand roles), so the log-joint is pass 1's bit for bit
//     and a cleared pair would give r = 0 exactly;
//   - r = 2^(ll2 - logZ2), Nk, sum r ||x_b||^2 and sum r S on the VALU, and
//     bf16(r)^T x_b on the matrix cores (r as the A operand, the rows read from LDS by
//     the transposing reads).
// The rows of the next tile are in flight while a tile is computed.  slab counts the
// partials of iso_bf16_accum's split (its slabs times its row groups), so either
// kernel fills the same partial slots.
__host__ __device__ constexpr int bf16_gather_rs(int DP) { return DP + 16; }   // bf16 row stride (odd x 32 bytes)
__host__ __device__ constexpr size_t bf16_gather_lds_bytes(int DP) {
  return (size_t)(DP / 16) * 64 * sizeof(bf16x8)                   // the block's mu operands
         + (size_t)kGatherWaves * 32 * bf16_gather_rs(DP) * 2       // x_b tile per wave
         + (size_t)kGatherWaves * 32 * sizeof(float2)               // row state per wave
         + (size_t)kGatherWaves * 64 * sizeof(int);                 // row queue per wave
}

template <int DP>
__global__ __attribute__((amdgpu_flat_work_group_size(64 * kGatherWaves, 64 * kGatherWaves),
                          amdgpu_waves_per_eu(gather_waves_per_simd(DP), gather_waves_per_simd(DP))))
void iso_bf16_gather(const float* __restrict__ X, int64_t ldx, int64_t N, int D,
                     const bf16x8* __restrict__ mu_op, const f32x4* __restrict__ kc, int KB, int KP,
                     const float2* __restrict__ rowstat, const unsigned* __restrict__ need,
                     const unsigned* __restrict__ needcount, int64_t dense_min, int nslab,
                     int64_t rows_per_slab, float* __restrict__ part_mu, float* __restrict__ part_nk,
                     float* __restrict__ part_sig, int dense) {
  constexpr int NC = DP / 16;
  constexpr int NJ = DP / 32;
  constexpr int RS = bf16_gather_rs(DP);
  constexpr int BLK = NC * 64;   // bf16x8 per component block
  static_assert(DP <= 128, "one contraction chain");
  if (need_total(needcount) >= dense_min) return;   // iso_bf16_accum runs instead (uniform exit)

  extern __shared__ __align__(16) unsigned char lds_raw[];
  unsigned char* lp = lds_raw;
  bf16x8* mu_l = reinterpret_cast<bf16x8*>(lp);     lp += (size_t)BLK * sizeof(bf16x8);
  __bf16* xt_all = reinterpret_cast<__bf16*>(lp);   lp += (size_t)kGatherWaves * 32 * RS * 2;
  float2* rs_all = reinterpret_cast<float2*>(lp);   lp += (size_t)kGatherWaves * 32 * sizeof(float2);
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
  float2* rs_l = rs_all + wave * 32;
  int* q_l = q_all + wave * 64;
  const f32x4 w = kc[(int64_t)kb * 32 + c];   // {c0, ish, 2 ish, ||mu||^2} of component c
  const float c0 = w.x, ish = w.y, ish2 = w.z, musq = w.w;

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
    queue_fill<(DP > 64)>(words, tb, t_begin, t_end, mword, mnext, jn, qt, qh, lane, c, g, q_l);
    const int cnt = qt - qh < 32 ? qt - qh : 32;
    asm volatile("s_waitcnt lgkmcnt(0)" ::: "memory");
    e = c < cnt ? q_l[(qh + c) & 63] : -1;
    qh += cnt;
    return cnt;
  };

  f32x4 raw[2 * NC];
  float2 rst;
  const bool xbuf = slab_fits(r_end > r_begin ? r_end - r_begin : 0, ldx);
  const bool xfull = xbuf && D == DP;
  const buf_rsrc xres = slab_rsrc(X, ldx, r_begin, xbuf && r_end > r_begin ? r_end : r_begin);
  const buf_rsrc rres = make_rsrc(rowstat + r_begin, (uint32_t)((r_end > r_begin ? r_end - r_begin : 0) * sizeof(float2)));
  auto issue = [&](int e) __attribute__((always_inline)) {
    const bool ok = e >= 0;
    if (xfull) {
      const int off = buf_off(ok ? (int)((int64_t)e * ldx * (int64_t)sizeof(float)) + 32 * g : kBufOob);
#pragma unroll
      for (int q = 0; q < NC; ++q) {
        raw[2 * q] = __builtin_bit_cast(f32x4, __builtin_amdgcn_raw_buffer_load_b128(xres, off, 64 * q, 0));
        raw[2 * q + 1] = __builtin_bit_cast(f32x4, __builtin_amdgcn_raw_buffer_load_b128(xres, off, 64 * q + 16, 0));
      }
    } else if (xbuf) {
#pragma unroll
      for (int q = 0; q < NC; ++q) {
        raw[2 * q] = slab_row4(xres, ldx, e, 16 * q + 8 * g, D, ok);
        raw[2 * q + 1] = slab_row4(xres, ldx, e, 16 * q + 8 * g + 4, D, ok);
      }
    } else {
      const int64_t row = r_begin + (ok ? e : 0);
#pragma unroll
      for (int q = 0; q < NC; ++q) {
        raw[2 * q] = load_row4(X, ldx, row, 16 * q + 8 * g, D, ok);
        raw[2 * q + 1] = load_row4(X, ldx, row, 16 * q + 8 * g + 4, D, ok);
      }
    }
    const float2 v = __builtin_bit_cast(
        float2, __builtin_amdgcn_raw_buffer_load_b64(rres, buf_off(ok ? e * (int)sizeof(float2) : kBufOob), 0, 0));
    rst = make_float2(ok ? v.x : INFINITY, v.y);   // a row past the queue: logZ2 = +inf, r = 0
  };

  f32x16 acc[NJ];
#pragma unroll
  for (int j = 0; j < NJ; ++j) acc[j] = zero16();
  float nk = 0.0f, srx = 0.0f, srs = 0.0f;

  int e;
  int cnt = take(e);
  if (cnt > 0) issue(e);
  while (cnt > 0) {
    // This tile's rows: bf16 in the A-operand layout, row-major to LDS, row state to LDS.
    bf16x8 xa[NC];
#pragma unroll
    for (int q = 0; q < NC; ++q) xa[q] = to_bf16x8(raw[2 * q], raw[2 * q + 1]);
    asm volatile("s_waitcnt lgkmcnt(0)" ::: "memory");   // the previous tile's LDS reads are done
#pragma unroll
    for (int q = 0; q < NC; ++q) *reinterpret_cast<bf16x8*>(xt + c * RS + 16 * q + 8 * g) = xa[q];
    if (g == 0) rs_l[c] = rst;
    int en;
    const int cnt_next = take(en);
    if (cnt_next > 0) issue(en);
    asm volatile("s_waitcnt lgkmcnt(0)" ::: "memory");

    // S = x_b mu_b^T: lane = component c, register i = row acc_row(i, g).
    f32x16 s = zero16();
#pragma unroll
    for (int q = 0; q < NC; ++q) s = mfma_bf16(xa[q], mu_l[q * 64 + lane], s);
    float r[16];
#pragma unroll
    for (int i = 0; i < 16; ++i) {
      const float2 z = rs_l[acc_row(i, g)];   // {logZ2, ||x_b||^2}
      const float ll = fmaf(ish2, s[i], fmaf(-ish, z.y, c0));
      const float rv = fast_exp2(ll - z.x);
      nk += rv;
      srx = fmaf(rv, z.y, srx);
      srs = fmaf(rv, s[i], srs);
      r[i] = rv;
    }
    bf16x8 a[2];
    acc_to_row_operands(r, a);
#pragma unroll
    for (int p = 0; p < 2; ++p) {
      // A step whose 16 rows of bf16(r) are all zero adds nothing.
      if (dense || any_nonzero(a[p])) {
#pragma unroll
        for (int j = 0; j < NJ; ++j) acc[j] = mfma_bf16(a[p], lds_rows_operand(xt, RS, 16 * p, 32 * j, lane), acc[j]);
      }
    }
    e = en;
    cnt = cnt_next;
  }

  nk += __shfl_xor(nk, 32);
  srx += __shfl_xor(srx, 32);
  srs += __shfl_xor(srs, 32);
  const int64_t kbase = (int64_t)slab * KP + (int64_t)kb * 32;
#pragma unroll
  for (int j = 0; j < NJ; ++j) {
#pragma unroll
    for (int i = 0; i < 16; ++i) part_mu[(kbase + acc_row(i, g)) * DP + 32 * j + c] = acc[j][i];
  }
  if (g == 0) {
    part_nk[kbase + c] = nk;
    part_sig[kbase + c] = fmaf(musq, nk, fmaf(-2.0f, srs, srx));
  }
}

template <int DP>
hipError_t launch_bf16(const IsoPlan& pl, const float* X, int64_t ldx, unsigned char* ws,
                       float* logZ, bool run1, bool run2, bool dense, hipStream_t stream) {
  const bf16x8* mu_op = reinterpret_cast<const bf16x8*>(ws + pl.off_musw);
  const f32x4* kc = reinterpret_cast<const f32x4*>(ws + pl.off_kcblk);
  float2* rowstat = reinterpret_cast<float2*>(ws + pl.off_rowstat);
  unsigned* ljmask = reinterpret_cast<unsigned*>(ws + pl.off_ljmask);
  unsigned* ljcount = reinterpret_cast<unsigned*>(ws + pl.off_ljcount);
  if (run1) {
    if (pl.bfneed) {
      if constexpr (DP <= 128) {
        const size_t lds1 = bf16_lse_lds_bytes<DP>() + (size_t)kWaves * 32 * pl.KB * 2;
        if (lds1 > 65536) {
          hipError_t e = hipFuncSetAttribute(reinterpret_cast<const void*>(&iso_bf16_lse<DP, true>),
                                             hipFuncAttributeMaxDynamicSharedMemorySize, (int)lds1);
          if (e != hipSuccess) return e;
        }
        hipLaunchKernelGGL((iso_bf16_lse<DP, true>), dim3((unsigned)cdiv(pl.N, 32 * kWaves)), dim3(kThreads), lds1,
                           stream, X, ldx, pl.N, (int)pl.D, mu_op, kc, pl.KB, logZ, rowstat, ljmask, ljcount,
                           dense ? 1 : 0);
      }
    } else {
      constexpr size_t lds1 = bf16_lse_lds_bytes<DP>();
      hipLaunchKernelGGL(iso_bf16_lse<DP>, dim3((unsigned)cdiv(pl.N, 32 * kWaves)), dim3(kThreads), lds1,
                         stream, X, ldx, pl.N, (int)pl.D, mu_op, kc, pl.KB, logZ, rowstat, ljmask, ljcount,
                         dense ? 1 : 0);
    }
  }
  if (!run2) return hipGetLastError();
  // With need masks: the gathering pass (one slab per partial of the dense split) when
  // fewer than 3/4 of the (row, block) pairs are needed, else iso_bf16_accum; both are
  // launched and the needed-pair count selects one on the device.
  const int64_t dense_min = cdiv(cdiv(pl.N, 32) * 32 * (int64_t)pl.KB * 3, 4);
  if (pl.bfneed) {
    if constexpr (DP <= 128) {
      constexpr size_t ldsg = bf16_gather_lds_bytes(DP);
      static_assert(ldsg <= 65536, "gathering tiles fit the default LDS allocation");
      hipLaunchKernelGGL(iso_bf16_gather<DP>, dim3((unsigned)gather_grid(pl.npart, pl.KB)),
                         dim3(64 * kGatherWaves), ldsg, stream, X, ldx, pl.N, (int)pl.D, mu_op, kc, pl.KB, pl.KP,
                         rowstat, ljmask, ljcount, dense_min, pl.npart, (int64_t)round_up(cdiv(pl.N, pl.npart), 32),
                         reinterpret_cast<float*>(ws + pl.off_part_mu), reinterpret_cast<float*>(ws + pl.off_part_nk),
                         reinterpret_cast<float*>(ws + pl.off_part_sig), dense ? 1 : 0);
    }
  }
  auto launch = [&](auto cb_tag) -> hipError_t {
    constexpr int CB = decltype(cb_tag)::value;
    constexpr size_t lds = bf16_accum_lds_bytes(DP, CB);
    if constexpr (!bf16_accum_fits(DP, CB)) {
      return hipErrorInvalidValue;   // never chosen by the plan
    } else {
      if (lds > 65536) {
        hipError_t e = hipFuncSetAttribute(reinterpret_cast<const void*>(&iso_bf16_accum<DP, CB>),
                                           hipFuncAttributeMaxDynamicSharedMemorySize, (int)lds);
        if (e != hipSuccess) return e;
      }
      hipLaunchKernelGGL((iso_bf16_accum<DP, CB>), dim3((unsigned)(pl.nslab * pl.ncg)), dim3(kAccThreads),
                         lds, stream, X, ldx, pl.N, (int)pl.D, mu_op, kc, pl.KB, pl.KP, rowstat,
                         pl.nslab, pl.rows_per_slab, reinterpret_cast<float*>(ws + pl.off_part_mu),
                         reinterpret_cast<float*>(ws + pl.off_part_nk),
                         reinterpret_cast<float*>(ws + pl.off_part_sig), dense ? 1 : 0,
                         pl.bfneed ? ljcount : nullptr, dense_min);
      return hipGetLastError();
    }
  };
  return pl.cpg == 1   ? launch(std::integral_constant<int, 1>{})
         : pl.cpg == 2 ? launch(std::integral_constant<int, 2>{})
                       : launch(std::integral_constant<int, 4>{});
}

// ---------------------------------------------------------------------------
// bf16 operand contract above D = 256 (any D).  A row's rounded operands no longer
// fit in registers, so pass 1 (iso_bf16_lse_wide) tiles the contraction over
// components: per tile of kBwCTB component blocks each wave re-reads its 32 rows
// (L2) chunk by chunk, rounds them to bf16 and accumulates S^T = mu_b . x_b^T for
// the tile's blocks, with the tile's operands staged in LDS: an fp32 chain per 256
// dimensions, added into an fp64 sum; S, ||x_b||^2 (fp64) and the constants are
// combined in fp64 and the fp32 log-joint is stored, [32-row tile][KP][32 rows].  Pass 2 (iso_bf16_accum_wide) reads r
// from it: bf16(r)^T bf16(X) per range of kBwDR dimensions on an X tile rounded to
// bf16 in LDS, Nk = sum r, and sig_acc = sum r ||x_b - mu||^2 with
// ish ||x_b - mu||^2 = c0' - ll2, c0' = c0 + ish ||mu||^2 (the log-joint's terms
// regrouped).  Calls whose log-joint exceeds kMaxLjBytes run as row chunks.
// ---------------------------------------------------------------------------
constexpr int kBwCTB = 4;    // component blocks per pass-1 tile
constexpr int kBwQS = 4;     // 16-dimension chunks per pass-1 stage
constexpr int kBwFlush = 4;  // stages per fp32 chain: its sum then joins an fp64 one
__host__ __device__ constexpr int bw_stage_ops() { return kBwCTB * kBwQS * 64; }   // bf16x8
__host__ __device__ constexpr size_t bw_lse_lds_bytes() {
  return (size_t)2 * (bw_stage_ops() * sizeof(bf16x8) + kBwCTB * 32 * sizeof(f32x4));
}

__global__ __launch_bounds__(kThreads) void iso_bf16_lse_wide(const float* __restrict__ X, int64_t ldx,
                                                              int64_t N, int D, int DP,
                                                              const bf16x8* __restrict__ mu_op,
                                                              const f32x4* __restrict__ kc, int KB, int KP,
                                                              float* __restrict__ logZ,
                                                              float2* __restrict__ rowstat,
                                                              float* __restrict__ lj) {
  constexpr int SO = bw_stage_ops();
  constexpr int LPT = SO / kThreads;
  static_assert(LPT == kBwCTB && kThreads == kBwQS * 64, "fetch register u holds block u of the tile");
  extern __shared__ __align__(16) unsigned char lds_raw[];
  bf16x8* mu_l = reinterpret_cast<bf16x8*>(lds_raw);                               // [2][SO]
  f32x4* kc_l = reinterpret_cast<f32x4*>(lds_raw + 2 * SO * sizeof(bf16x8));       // [2][CTB * 32]

  const int NQ = DP / 16, nst = NQ / kBwQS;
  const int ntile = (KB + kBwCTB - 1) / kBwCTB;
  const int tid = threadIdx.x, lane = tid & 63;
  const int wave = __builtin_amdgcn_readfirstlane(tid >> 6);
  const int c = lane & 31, g = lane >> 5;
  const int64_t tile = (int64_t)blockIdx.x * kWaves + wave;
  const int64_t row = tile * 32 + c;
  const bool valid = row < N;
  const int64_t nstage = (int64_t)ntile * nst;

  bf16x8 st[LPT];
  f32x4 kst = {-INFINITY, 0.0f, 0.0f, 0.0f};
  auto fetch = [&](int64_t s) {
    const int t = (int)(s / nst), qs = (int)(s % nst);
    const int kb0 = t * kBwCTB;
    const int cnt = KB - kb0 < kBwCTB ? KB - kb0 : kBwCTB;
    const int qq = tid >> 6;
#pragma unroll
    for (int u = 0; u < LPT; ++u) {
      if (u < cnt) {
        st[u] = mu_op[((int64_t)(kb0 + u) * NQ + kBwQS * qs + qq) * 64 + lane];
      } else {
#pragma unroll
        for (int e = 0; e < 8; ++e) st[u][e] = (__bf16)0.0f;
      }
    }
    if (tid < kBwCTB * 32) kst = tid < cnt * 32 ? kc[(int64_t)kb0 * 32 + tid] : f32x4{-INFINITY, 0.0f, 0.0f, 0.0f};
  };
  auto commit = [&](int buf) {
#pragma unroll
    for (int u = 0; u < LPT; ++u) mu_l[buf * SO + u * kThreads + tid] = st[u];
    if (tid < kBwCTB * 32) kc_l[buf * kBwCTB * 32 + tid] = kst;
  };
  // This lane's row, dimensions 16q + 8g .. +7 of the stage's chunks.
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

  // S of the tile's blocks: an fp32 chain over kBwFlush stages (256 dimensions),
  // then added to an fp64 sum, so no fp32 chain grows past ~1/4 of S at D ~ 1000.
  f32x16 acc[kBwCTB];
  double sacc[kBwCTB][16];
#pragma unroll
  for (int u = 0; u < kBwCTB; ++u) {
    acc[u] = zero16();
#pragma unroll
    for (int i = 0; i < 16; ++i) sacc[u][i] = 0.0;
  }
  // This half's sum of squares (fp64: a sequential fp32 sum over D ~ 1000 terms
  // of ~4 each would carry ~4e-3), then the row's.
  double xsq = 0.0, xsqf = 0.0;
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
    bf16x8 xb[kBwQS];
#pragma unroll
    for (int qq = 0; qq < kBwQS; ++qq) xb[qq] = to_bf16x8(raw[2 * qq], raw[2 * qq + 1]);
    if (t == 0) {
#pragma unroll
      for (int qq = 0; qq < kBwQS; ++qq) {
#pragma unroll
        for (int e = 0; e < 8; ++e) {
          const double v = (double)(float)xb[qq][e];
          xsq = fma(v, v, xsq);
        }
      }
    }
    if (more) {
      fetch(s + 1);
      loadx(s + 1);
    }
    const bf16x8* mp = mu_l + buf * SO + lane;
#pragma unroll
    for (int u = 0; u < kBwCTB; ++u) {
      if (u < cnt) {
#pragma unroll
        for (int qq = 0; qq < kBwQS; ++qq) acc[u] = mfma_bf16(mp[(u * kBwQS + qq) * 64], xb[qq], acc[u]);
      }
    }
    if ((qs + 1) % kBwFlush == 0 || qs == nst - 1) {
#pragma unroll
      for (int u = 0; u < kBwCTB; ++u) {
#pragma unroll
        for (int i = 0; i < 16; ++i) sacc[u][i] += (double)acc[u][i];
        acc[u] = zero16();
      }
    }
    if (qs == nst - 1) {   // the tile's blocks are complete: S^T, lane = row, register i = component
      if (t == 0) xsqf = xsq + __shfl_xor(xsq, 32);
      const f32x4* kp = kc_l + buf * kBwCTB * 32;
      float bm = -INFINITY;
      float ll[kBwCTB][16];
#pragma unroll
      for (int u = 0; u < kBwCTB; ++u) {
#pragma unroll
        for (int i = 0; i < 16; ++i) {
          // c0 - ish ||x_b||^2 + 2 ish S with the terms (each ~4 D log2 units on
          // clustered data) combined in fp64, rounded once.
          const f32x4 w = kp[u * 32 + acc_row(i, g)];
          ll[u][i] = (float)(((double)w.x - (double)w.y * xsqf) + (double)w.z * sacc[u][i]);
          sacc[u][i] = 0.0;
          if (u < cnt) {
            if (valid) ljr[((int64_t)(kb0 + u) * 32 + acc_row(i, g)) * 32] = ll[u][i];
            bm = fmaxf(bm, ll[u][i]);
          }
        }
      }
      const float mn = fmaxf(mx, bm);
      const float ms = (mn == -INFINITY) ? 0.0f : mn;
      float a = sm * fast_exp2(mx - ms);
#pragma unroll
      for (int u = 0; u < kBwCTB; ++u) {
        if (u < cnt) {
#pragma unroll
          for (int i = 0; i < 16; ++i) a += fast_exp2(ll[u][i] - ms);
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
    rowstat[row] = make_float2(lz2, (float)xsqf);
    if (logZ) logZ[row] = lz2 * (float)kLn2;
  }
}

// Pass 2: one workgroup per (row slab, group of kBwCB component blocks, range of
// kBwDR dimensions); wave u owns block cg kBwCB + u and every column of the range (8
// tiles of 32).  Per 32-row tile the workgroup stages the rows' range of X rounded
// to bf16 (row-major, stride kBwDR + 16: an odd multiple of 32 bytes, as the
// transposing reads want) and their {logZ2, ||x_b||^2}; each lane forms r for its
// component (lane % 32) and the 8 rows of each 16-row step its half-wave supplies,
// which is the A-operand layout of bf16(r)^T X, so no exchange is needed.  The waves
// of range 0 also sum Nk and r (c0' - ll2).
__host__ __device__ constexpr int bw_xr() { return kBwDR + 16; }
__host__ __device__ constexpr size_t bw_accum_lds_bytes() {
  return (size_t)2 * 32 * bw_xr() * sizeof(__bf16) + (size_t)2 * 32 * sizeof(float2);
}

__global__ __attribute__((amdgpu_flat_work_group_size(64 * kBwCB, 64 * kBwCB), amdgpu_waves_per_eu(2, 2)))
void iso_bf16_accum_wide(const float* __restrict__ X, int64_t ldx, int64_t N, int D, int DP,
                         const f32x4* __restrict__ kc, int KB, int KP, const float2* __restrict__ rowstat,
                         const float* __restrict__ lj, int nslab, int64_t rows_per_slab, int ncg, int ndr,
                         float* __restrict__ part_mu, float* __restrict__ part_nk,
                         float* __restrict__ part_sig, int dense) {
  constexpr int T = 64 * kBwCB;
  constexpr int XR = bw_xr();
  constexpr int NJ = kBwDR / 32;
  constexpr int LPT = 32 * (kBwDR / 4) / T;   // float4 of the X tile per thread
  static_assert(LPT * T == 32 * kBwDR / 4, "even split");
  extern __shared__ __align__(16) unsigned char lds_raw[];
  __bf16* xr = reinterpret_cast<__bf16*>(lds_raw);                      // [2][32][XR]
  float2* rs = reinterpret_cast<float2*>(xr + 2 * 32 * XR);              // [2][32]

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
  f32x4 w = {-INFINITY, 0.0f, 0.0f, 0.0f};
  if (active) w = kc[comp];
  const float c0p = (float)((double)w.x + (double)w.y * (double)w.w);   // c0 + ish ||mu||^2

  f32x4 stage[LPT];
  float2 rstage = make_float2(INFINITY, 0.0f);
  auto fetch = [&](int t) {
    const int64_t row0 = r_begin + (int64_t)t * 32;
#pragma unroll
    for (int q = 0; q < LPT; ++q) {
      const int idx = q * T + tid;
      const int64_t rw = row0 + idx / (kBwDR / 4);
      stage[q] = load_row4(X, ldx, rw, col0 + (idx % (kBwDR / 4)) * 4, D, rw < r_end);
    }
    if (tid < 32) rstage = row0 + tid < r_end ? rowstat[row0 + tid] : make_float2(INFINITY, 0.0f);
  };
  auto commit = [&](int buf) {
    __bf16* dst = xr + buf * 32 * XR;
#pragma unroll
    for (int q = 0; q < LPT; ++q) {
      const int idx = q * T + tid;
      const f32x4 v = stage[q];
      typedef __bf16 bf16x4 __attribute__((ext_vector_type(4)));
      const bf16x4 b = {(__bf16)v.x, (__bf16)v.y, (__bf16)v.z, (__bf16)v.w};
      *reinterpret_cast<bf16x4*>(dst + (idx / (kBwDR / 4)) * XR + (idx % (kBwDR / 4)) * 4) = b;
    }
    if (tid < 32) rs[buf * 32 + tid] = rstage;
  };

  f32x16 acc[NJ];
#pragma unroll
  for (int j = 0; j < NJ; ++j) acc[j] = zero16();
  float nk = 0.0f, sg = 0.0f;
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
      const float2* rt = rs + buf * 32;
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
          const bool in = row0 + rr < r_end;   // rows past N hold no log-joint
          const float l = in ? lv[e] : c0p;
          const float rv = in ? fast_exp2(l - rt[rr].x) : 0.0f;
          r8[e] = rv;
          if (stats) {
            nk += rv;
            sg = fmaf(rv, c0p - l, sg);
          }
        }
        a[p] = to_bf16x8(f32x4{r8[0], r8[1], r8[2], r8[3]}, f32x4{r8[4], r8[5], r8[6], r8[7]});
      }
      const __bf16* xt = xr + buf * 32 * XR;
#pragma unroll
      for (int p = 0; p < 2; ++p) {
        // A step whose 16 rows x 32 components of bf16(r) are all zero adds nothing.
        if (dense || any_nonzero(a[p])) {
#pragma unroll
          for (int j = 0; j < NJ; ++j) acc[j] = mfma_bf16(a[p], lds_rows_operand(xt, XR, 16 * p, 32 * j, lane), acc[j]);
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
      for (int i = 0; i < 16; ++i) part_mu[(kbase + acc_row(i, g)) * DP + col] = acc[j][i];
    }
  }
  if (dr == 0) {
    nk += __shfl_xor(nk, 32);
    sg += __shfl_xor(sg, 32);
    if (g == 0) {
      part_nk[kbase + c] = nk;
      part_sig[kbase + c] = w.y > 0.0f ? sg / w.y : 0.0f;
    }
  }
}

hipError_t launch_bf16_wide(const IsoPlan& pl, const float* X, int64_t ldx, unsigned char* ws, float* logZ,
                            bool run1, bool run2, bool dense, hipStream_t stream) {
  const bf16x8* mu_op = reinterpret_cast<const bf16x8*>(ws + pl.off_musw);
  const f32x4* kc = reinterpret_cast<const f32x4*>(ws + pl.off_kcblk);
  float2* rowstat = reinterpret_cast<float2*>(ws + pl.off_rowstat);
  float* lj = reinterpret_cast<float*>(ws + pl.off_lj);
  if (run1) {
    constexpr size_t lds1 = bw_lse_lds_bytes();
    static_assert(lds1 <= 65536, "pass-1 stages fit the default LDS allocation");
    hipLaunchKernelGGL(iso_bf16_lse_wide, dim3((unsigned)cdiv(pl.N, 32 * kWaves)), dim3(kThreads), lds1, stream,
                       X, ldx, pl.N, (int)pl.D, pl.DP, mu_op, kc, pl.KB, pl.KP, logZ, rowstat, lj);
  }
  if (!run2) return hipGetLastError();
  constexpr size_t lds2 = bw_accum_lds_bytes();
  static_assert(lds2 <= 65536, "pass-2 tiles fit the default LDS allocation");
  hipLaunchKernelGGL(iso_bf16_accum_wide, dim3((unsigned)((int64_t)pl.nslab * pl.ncg * pl.ndr)), dim3(64 * kBwCB),
                     lds2, stream, X, ldx, pl.N, (int)pl.D, pl.DP, kc, pl.KB, pl.KP, rowstat, lj, pl.nslab,
                     pl.rows_per_slab, pl.ncg, pl.ndr, reinterpret_cast<float*>(ws + pl.off_part_mu),
                     reinterpret_cast<float*>(ws + pl.off_part_nk), reinterpret_cast<float*>(ws + pl.off_part_sig),
                     dense ? 1 : 0);
  return hipGetLastError();
}

}  // namespace
}  // namespace fgmm

using namespace fgmm;

namespace {
// Rows per call of the bf16 contract above D = 256, whose log-joint must fit
// kMaxLjBytes: a multiple of 128 rows.  Larger calls run in chunks of this many rows.
int64_t iso_bw_chunk_rows(int64_t K) {
  const int64_t KP = round_up(K < 1 ? 1 : K, 32);
  return (int64_t)(kMaxLjBytes / ((size_t)KP * 32 * sizeof(float))) / 4 * 4 * 32;
}
bool iso_bw_call(int64_t D, unsigned flags) {
  return (flags & FGMM_FLAG_BF16) != 0 && iso_bf16_wide(iso_padded_dim(D));
}
}  // namespace

extern "C" size_t fgmm_iso_workspace_bytes(int64_t N, int64_t K, int64_t D) {
  if (N < 0 || K < 0 || D < 1) return 0;
  return make_plan(N, K, D, false).total;
}

extern "C" size_t fgmm_iso_workspace_bytes_ex(int64_t N, int64_t K, int64_t D, unsigned flags) {
  if (N < 0 || K < 0 || D < 1) return 0;
  const int64_t rows = iso_bw_call(D, flags) ? std::min(N, iso_bw_chunk_rows(K)) : N;
  return make_plan(rows, K, D, wants_stored_lj(flags), (flags & FGMM_FLAG_BF16) != 0, wants_auto_lj(flags)).total;
}

extern "C" int fgmm_iso_estep_f32(const float* X, int64_t ldx, int64_t N, int64_t D, const float* mu,
                                  int64_t ldmu, int64_t K, const float* log_sigma_sq,
                                  const float* log_pi, float* logZ, float* Nk, float* mu_acc,
                                  float* sig_acc, void* workspace, size_t workspace_bytes,
                                  unsigned flags, void* stream_) {
  hipStream_t stream = reinterpret_cast<hipStream_t>(stream_);
  const bool want_logz = !(flags & FGMM_FLAG_NO_LOGZ);
  const bool accumulate = (flags & FGMM_FLAG_ACCUMULATE) != 0;
  const bool atomic = (flags & FGMM_FLAG_ATOMIC_REDUCE) != 0;
  const bool dense = (flags & FGMM_FLAG_DENSE) != 0;
  if (N < 0 || K < 0 || D < 1) return FGMM_ERR_INVALID_ARG;
  if (N > 0 && (X == nullptr || ldx < round_up(D, 4) || (ldx % 4) != 0 ||
                (reinterpret_cast<uintptr_t>(X) & 15) != 0))
    return FGMM_ERR_INVALID_ARG;
  if (N > 0 && want_logz && logZ == nullptr) return FGMM_ERR_INVALID_ARG;
  if (K > 0 && (mu == nullptr || ldmu < D || log_sigma_sq == nullptr || log_pi == nullptr ||
                Nk == nullptr || mu_acc == nullptr || sig_acc == nullptr))
    return FGMM_ERR_INVALID_ARG;
  if (N > kMaxRows || K > (int64_t)1 << 24) return FGMM_ERR_UNSUPPORTED;
  const bool bf16 = (flags & FGMM_FLAG_BF16) != 0;
  if (iso_bw_call(D, flags) && K > 0 && N > iso_bw_chunk_rows(K)) {
    // The bf16 contract above D = 256 stores the log-joint, at most kMaxLjBytes per
    // call: larger N runs as consecutive row chunks on one workspace, each chunk after
    // the first adding its statistics to the outputs.  A phase split cannot span them.
    if (flags & (FGMM_FLAG_PHASE1 | FGMM_FLAG_PHASE2)) return FGMM_ERR_UNSUPPORTED;
    const int64_t rows = iso_bw_chunk_rows(K);
    for (int64_t r0 = 0; r0 < N; r0 += rows) {
      const int64_t n = std::min(rows, N - r0);
      const unsigned f = r0 == 0 ? flags : (flags | FGMM_FLAG_ACCUMULATE);
      const int st = fgmm_iso_estep_f32(X + r0 * ldx, ldx, n, D, mu, ldmu, K, log_sigma_sq, log_pi,
                                        logZ ? logZ + r0 : nullptr, Nk, mu_acc, sig_acc, workspace,
                                        workspace_bytes, f, stream_);
      if (st != FGMM_OK) return st;
    }
    return FGMM_OK;
  }
  // The stored log-joint path streams X with 32-bit buffer offsets (row stride at
  // most kMaxBufLdx floats); wider strides recompute, which needs less workspace.
  const IsoPlan pl = make_plan(N, K, D, wants_stored_lj(flags) && ldx <= kMaxBufLdx, bf16, wants_auto_lj(flags));
  if (workspace_bytes < pl.total || (pl.total > 0 && workspace == nullptr)) return FGMM_ERR_WORKSPACE;
  if (!want_logz) logZ = nullptr;
  unsigned char* ws = static_cast<unsigned char*>(workspace);
  const bool sel1 = (flags & FGMM_FLAG_PHASE1) != 0, sel2 = (flags & FGMM_FLAG_PHASE2) != 0;
  const bool run1 = sel1 || !sel2, run2 = sel2 || !sel1;

  if (K == 0) {
    // No components: logsumexp over an empty set is -inf (flash_gmm.py:72-73,102).
    if (N > 0 && logZ)
      hipLaunchKernelGGL(fill_f32, dim3((unsigned)cdiv(N, 256)), dim3(256), 0, stream, logZ, N,
                         -INFINITY);
    return hipGetLastError() == hipSuccess ? FGMM_OK : FGMM_ERR_HIP;
  }

  if (run1 && bf16)
    hipLaunchKernelGGL(iso_bf16_prep, dim3(pl.KB), dim3(64), 0, stream, mu, ldmu, K, (int)D, pl.DP,
                       log_sigma_sq, log_pi, reinterpret_cast<bf16x8*>(ws + pl.off_musw),
                       reinterpret_cast<f32x4*>(ws + pl.off_kcblk),
                       pl.bfneed ? reinterpret_cast<unsigned*>(ws + pl.off_ljcount) : nullptr);
  else if (run1)
    hipLaunchKernelGGL(iso_prep, dim3(pl.KB), dim3(64), 0, stream, mu, ldmu, K, (int)D, pl.DP,
                       log_sigma_sq, log_pi, reinterpret_cast<double2*>(ws + pl.off_kcblk),
                       reinterpret_cast<double4*>(ws + pl.off_kclin),
                       reinterpret_cast<double4*>(ws + pl.off_kcgat),
                       reinterpret_cast<bf16x8*>(ws + pl.off_mu3),
                       (pl.lj || pl.need) ? reinterpret_cast<unsigned*>(ws + pl.off_ljcount) : nullptr);
  if (N > 0) {
    auto run = [&](auto dp_tag) -> hipError_t {
      constexpr int DP = decltype(dp_tag)::value;
      return bf16 ? launch_bf16<DP>(pl, X, ldx, ws, logZ, run1, run2, dense, stream)
                  : launch_passes<DP>(pl, X, ldx, ws, logZ, run1, run2, dense, stream);
    };
    hipError_t e = hipSuccess;
    if (pl.bfw) {
      e = launch_bf16_wide(pl, X, ldx, ws, logZ, run1, run2, dense, stream);
    } else if (!bf16 && pl.DP > 128) {
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
  const float* pmu = reinterpret_cast<const float*>(ws + pl.off_part_mu);
  const float* pnk = reinterpret_cast<const float*>(ws + pl.off_part_nk);
  const float* psig = reinterpret_cast<const float*>(ws + pl.off_part_sig);
  const int64_t nout = K * (D + 2);
  if (atomic) {
    if (!accumulate) {
      hipLaunchKernelGGL(fill_f32, dim3((unsigned)cdiv(K, 256)), dim3(256), 0, stream, Nk, K, 0.0f);
      hipLaunchKernelGGL(fill_f32, dim3((unsigned)cdiv(K * D, 256)), dim3(256), 0, stream, mu_acc,
                         K * D, 0.0f);
      hipLaunchKernelGGL(fill_f32, dim3((unsigned)cdiv(K, 256)), dim3(256), 0, stream, sig_acc, K,
                         0.0f);
    }
    if (pl.npart > 0)
      hipLaunchKernelGGL(iso_reduce_atomic, dim3((unsigned)cdiv(nout, 256), (unsigned)pl.npart),
                         dim3(256), 0, stream, pmu, pnk, psig, pl.npart, pl.KP, pl.DP, K, (int)D, Nk,
                         mu_acc, sig_acc);
  } else if (pl.npart >= kWideReduce) {
    hipLaunchKernelGGL(iso_reduce_wide, dim3((unsigned)cdiv(nout, 4)), dim3(256), 0, stream, pmu, pnk,
                       psig, pl.npart, pl.KP, pl.DP, K, (int)D, Nk, mu_acc, sig_acc,
                       accumulate ? 1 : 0);
  } else {
    hipLaunchKernelGGL(iso_reduce, dim3((unsigned)cdiv(nout, 256)), dim3(256), 0, stream, pmu, pnk,
                       psig, pl.npart, pl.KP, pl.DP, K, (int)D, Nk, mu_acc, sig_acc,
                       accumulate ? 1 : 0);
  }
  return hipGetLastError() == hipSuccess ? FGMM_OK : FGMM_ERR_HIP;
}
