// Full-covariance GMM E-step for gfx950 (1 <= D <= 4096).
//
// Math (reference: flash_gmm_full_h100.py:289-296 constants, :103-130 pass 1,
// :171-228 pass 2), with L_k lower-triangular, L_k L_k^T = Sigma_k^-1, in log2 units:
//   b_k   = L_k^T mu_k
//   c_k   = (lpi_k + sum_d log(|L_k,dd| + 1e-30) - 0.5*D*log(2pi)) * log2(e)
//   v     = L_k^T x_n - b_k,   maha_nk = ||v||^2,   ll2_nk = c_k - 0.5*log2(e)*maha_nk
//   r_nk  = 2^(ll2_nk - logZ2_n)
//   Nk_k = sum_n r_nk;  mu_acc_k = sum_n r_nk x_n;  sig_outer_k = sum_n r_nk x_n x_n^T
//
// Pass 1 (full_lse_x6) whitens on the bf16 matrix cores in a centred split-bf16
// form: V^T = L_k^T X^T - b_k with each 16-dimension chunk contributing
// L_k[q]^T (x - mu_k)[q] to an fp32 accumulator, the offsets returned in fp64; each
// lane owns one row and 16 whitened coordinates per 32-row block of V^T, so maha is
// an in-lane fp64 sum plus one cross-half exchange.
//
// Default plan (workspace O(N + K D^2 + N K / 32 bits)): pass 1 leaves logZ2 per row
// and one need bit per (row, component); pass 2 (full_accum_gather) recomputes the
// whitening, bit for bit as pass 1 formed it, for the needed pairs only.  With
// FGMM_FLAG_STORE_LOGJOINT pass 1 stores the fp32 log-joint (N x K) and pass 2
// (full_accum) reads it.
//
// Pass 2 accumulates sig_outer as sum_rows (r x)(x^T) on fp32 MFMA with the r-scaled
// rows as the A operand.  Only the upper 32x32 blocks (d1 block <= d2 block) are
// accumulated; the finish mirrors them.  mu_acc is the running sum of the same
// r-scaled operands.

#include "fgmm_common.hpp"

#include <math.h>

#include <algorithm>
#include <type_traits>

namespace fgmm {
namespace {

constexpr int kWaves = 4;
constexpr int kGatherWaves = 4;                           // waves (row slabs) per gathering workgroup
constexpr int kThreads = 64 * kWaves;
constexpr int kAccWaves = 8;
constexpr int kAccThreads = 64 * kAccWaves;
constexpr int kCompsPerWG = 4;
constexpr int kRowGroups = 2;

struct FullPlan {
  int64_t N, K, D;
  int DP;       // D padded to 32
  int NMB;      // 32-row blocks of V^T (DP / 32)
  int NSB;      // upper 32x32 blocks of sig_outer: NMB*(NMB+1)/2
  int KP;       // K padded to kCompsPerWG
  int ncg, nslab, rgroups, npart;
  int64_t rows_per_slab;
  bool lj;      // pass 1 stores the log-joint; pass 2 reads it
  bool bf16;    // bf16 operand contract (FGMM_FLAG_BF16); always stores the log-joint
  bool need;    // default plan: pass 1 leaves need masks, pass 2 gathers
  int needmode; // how pass 1 forms the need masks: kNeedLists, kNeedBounds or kNeedRunMax
  bool wide;    // D > 256: full_lse_wide stores the log-joint, full_accum_wide reads it
  bool keep_lj; // 128 < D <= 256, default plan: pass 1 also stores the log-joint, and the
                // gathering pass 2 reads r from it instead of whitening the needed rows
  int nstrip;   // wide pass 2: strips of upper sig_outer blocks (one wave each)
  int ngrp;     // waves per (slab, component) in the gathering pass 2 (groups of sig blocks)
  int grid1;    // pass-1 workgroups with need masks (a persistent grid)
  bool autolj;  // default plan with a stored branch that a row-sample probe selects on the device
                // (FGMM_FLAG_STORE_LOGJOINT_AUTO, D <= 64): pass 1 also keeps the log-joint, and
                // full_accum_ljt reads r from it over the same slabs and partials
  int nprobe;   // the probe's sampled tiles
  size_t off_probe;
  size_t off_lop, off_bsw, off_ck, off_l3, off_esw, off_rowstat, off_part_sig, off_part_mu, off_part_nk,
      off_lj, off_need, off_bound, total;
};

// One LDS stage holds SMB 32-coordinate blocks of one component: all of them up to
// D = 64, one above (a whole component's operands, 72 or 128 KiB, would not fit twice).
__host__ __device__ constexpr int full_x6_smb(int DP) { return DP <= 64 ? DP / 32 : 1; }
__host__ __device__ constexpr int full_x6_stage(int DP) { return full_x6_smb(DP) * (DP / 16) * 4 * 64; }   // bf16x8
__host__ __device__ constexpr size_t full_x6_lds_bytes(int DP) {
  return (size_t)2 * full_x6_stage(DP) * sizeof(bf16x8) + (size_t)2 * (32 * full_x6_smb(DP) + 8) * sizeof(double);
}
constexpr size_t kFullLds = 160 * 1024;   // LDS per compute unit

// Need masks of the full model are per (32-row tile, component); pass 1 runs a
// persistent grid of grid1 workgroups and forms them in one of three ways:
//   kNeedLists:  each row keeps a list of candidates: the components within
//                kLjSkipGap of the row's running maximum when they were formed, each
//                with a bf16 upper bound of its log-joint.  The first
//                full_list_cands of a row sit in LDS, the rest of its kNeedListCap in
//                the wave's slot of the workspace, reused tile after tile; a candidate
//                past those sets its bit at once.  Once logZ2 is final the listed candidates are tested as
//                need_put_masks tests, into mask words in LDS.  On clustered data a row
//                has a few tens of candidates, so the workspace sees a few bytes per
//                row.  Used where the LDS lists and words fit beside the operand
//                stages.
//   kNeedBounds: each wave has a slot of TPW x 32 x KP bf16 bounds in the workspace,
//                reused tile after tile (up to kNeedExactMaxK components).
//   kNeedRunMax: the bit is set when the component is within kLjSkipGap of the running
//                maximum.
// The first two give the exact bits (the first unless a row has more than
// kNeedListCap candidates); otherwise a superset of them.  A pair outside
// the exact set has responsibility exactly 0, so the outputs are the same bits in every
// form.
constexpr int kNeedExactMaxK = 1024;
constexpr int kNeedRunMax = 0, kNeedBounds = 1, kNeedLists = 2;
constexpr int kNeedListCap = 64;   // listed candidates per row
// 32-row tiles per pass-1 wave: two up to D = 64, where the wave's registers hold both
// tiles' split rows, so that each operand read from LDS serves 64 rows and the
// operand set streams through the XCD's L2 half as many times.
__host__ __device__ constexpr int full_x6_tpw(int DP) { return DP <= 64 ? 2 : 1; }
// Candidates per row in LDS (the rest of a list is in the workspace).
__host__ __device__ constexpr int full_list_cands(int DP) { return full_x6_tpw(DP) == 2 ? 4 : 16; }
// Per wave: the LDS candidates of its rows, then a mask word per (tile, component).
__host__ __device__ constexpr size_t full_list_lds_bytes(int DP, int KP) {
  return (size_t)kWaves * full_x6_tpw(DP) * ((size_t)full_list_cands(DP) * 32 + (size_t)KP) * sizeof(unsigned);
}
// Candidates per row in the workspace.
__host__ __device__ constexpr int full_list_spill(int DP, int K) {
  return (K < kNeedListCap ? K : kNeedListCap) > full_list_cands(DP)
             ? (K < kNeedListCap ? K : kNeedListCap) - full_list_cands(DP)
             : 0;
}

// The stored branch of FGMM_FLAG_STORE_LOGJOINT_AUTO runs up to D = 64 (sig_outer's
// accumulators and split operands of one component fit a wave's registers).
__host__ __device__ constexpr bool flj_applies(int DP) { return DP <= 64; }

// Stored log-joint of the full model: per (32-row tile, component) 32 floats, rows
// contiguous, [tile][KP][32]; the tiles of the pass-1 grid (rounded up to 8, a
// workgroup's tiles with two per wave).  Pass 2 reads it unless recomputation is requested or it would exceed
// kMaxLjBytes: recomputing costs a D x D whitening per (row, component).
__host__ inline size_t full_lj_bytes(int64_t N, int KP) {
  return (size_t)round_up(cdiv(N, 32), 8) * (size_t)KP * 32 * sizeof(float);
}

// The gathering pass 2 holds the accumulators of the upper 32x32 blocks of sig_outer
// it owns in registers, with the rows' split operands: above D = 128 the blocks are
// dealt to this many waves per (slab, component), each recomputing the whitening.
__host__ __device__ constexpr int gather_sig_groups(int DP) {
  return DP <= 128 ? 1 : DP <= 160 ? 2 : DP <= 224 ? 3 : 4;
}
// Pass 1 and the gathering pass 2 run one wave per SIMD above D = 128 (the rows'
// split operands alone take 12 registers per 16 dimensions).
__host__ __device__ constexpr int full_waves_per_eu(int DP) { return DP <= 128 ? 2 : 1; }

// Above D = 256 (up to kFullMaxD) a row's split operands no longer fit in registers.
// Pass 1 (full_lse_wide) re-reads and re-splits each row for every group of
// kWideCG coordinate blocks and stores the log-joint; pass 2 (full_accum_wide)
// reads r from it, so the whitening is formed once per (row, component), and
// accumulates sig_outer in strips of up to kWideSW upper 32x32 blocks of one block
// row, one wave per (slab, component, strip).  Row counts whose log-joint would
// exceed kMaxLjBytes run as row chunks, as the bf16 contract does.
constexpr int kFullMaxD = 4096;
constexpr int kWideCG = 4;       // 32-coordinate blocks per pass-1 group
constexpr int kWideWaves1 = 8;   // waves (32-row tiles) per pass-1 workgroup
constexpr int kWideSW = 8;       // upper sig blocks per pass-2 strip
constexpr int kWideWaves2 = 4;   // strips per pass-2 workgroup
__host__ __device__ constexpr bool full_is_wide(int DP) { return DP > 256; }
// Partials of the wide pass 2 (slabs x KP x NSB x 4 KiB) are capped at this size.
constexpr size_t kWidePartBytes = (size_t)1 << 30;
__host__ __device__ inline int wide_strips(int NMB) {
  int s = 0;
  for (int b1 = 0; b1 < NMB; ++b1) s += (NMB - b1 + kWideSW - 1) / kWideSW;
  return s;
}

// Pass-2 layout of the bf16 contract (defined with its kernels below).
__host__ __device__ constexpr int bf16_comps_per_wg(int NMB);
__host__ __device__ constexpr int bf16_comp_reps(int NMB);
__host__ __device__ constexpr int bf16_row_groups(int NMB);

FullPlan make_plan(int64_t N, int64_t K, int64_t D, bool allow_lj = false, bool bf16 = false,
                   bool auto_lj = false) {
  FullPlan p{};
  p.N = N; p.K = K; p.D = D;
  p.DP = (int)round_up(D < 1 ? 1 : D, 32);
  p.NMB = p.DP / 32;
  p.NSB = p.NMB * (p.NMB + 1) / 2;
  p.KP = (int)round_up(K, kCompsPerWG);
  p.bf16 = bf16;
  p.wide = !bf16 && full_is_wide(p.DP);
  // The stored log-joint (and with it the bf16 contract) up to D = 128; above
  // D = 256 always (the entry point chunks the rows to keep it within kMaxLjBytes).
  p.lj = p.wide ? K > 0
                : (allow_lj || bf16) && K > 0 && p.DP <= 128 && full_lj_bytes(N, p.KP) <= kMaxLjBytes;
  p.need = !bf16 && !p.lj && K > 0;
  // Above D = 128 the gathering pass 2 runs as 2-4 launches (groups of sig_outer
  // blocks), each of which would whiten the needed rows again; 4 bytes per (row,
  // component) of stored log-joint replace those D x D whitenings.
  p.keep_lj = p.need && p.DP > 128 && !p.wide && full_lj_bytes(N, p.KP) <= kMaxLjBytes;
  p.autolj = p.need && auto_lj && flj_applies(p.DP) && N > 0 && K <= kProbeMaxKB &&
             full_lj_bytes(N, p.KP) <= kMaxLjBytes;
  p.nprobe = p.autolj ? (int)std::min<int64_t>(kProbeTiles, cdiv(N, 32)) : 0;
  // A list entry holds the component in 16 bits (the LDS limit keeps K far below that).
  p.needmode = !p.need ? kNeedRunMax
               : p.KP < 65536 &&
                         full_x6_lds_bytes(p.DP) + full_list_lds_bytes(p.DP, p.KP) <= kFullLds / full_waves_per_eu(p.DP)
                   ? kNeedLists
                   : K <= kNeedExactMaxK ? kNeedBounds : kNeedRunMax;
  p.ngrp = gather_sig_groups(p.DP);
  if (bf16) {
    p.ncg = (int)cdiv(K, (int64_t)bf16_comps_per_wg(p.NMB) * bf16_comp_reps(p.NMB));
    p.rgroups = bf16_row_groups(p.NMB);
  } else if (p.need) {
    p.ncg = (int)K;   // one wave per (row slab, component)
    p.rgroups = 1;
  } else if (p.wide) {
    p.nstrip = wide_strips(p.NMB);
    p.ncg = (int)K;
    p.rgroups = 1;
  } else {
    p.ncg = p.KP / kCompsPerWG;
    p.rgroups = kRowGroups;
  }
  const int64_t tile_rows = 32 * p.rgroups;
  if (p.need && N > 0) {
    // The gathering pass 2: about two rounds of waves at two waves per SIMD (each
    // slab holds a partial of D x D per component, so no more slabs than that).
    const int64_t want = gather_slab_count(cdiv((int64_t)8 * current_device_cus(), K * p.ngrp), cdiv(N, 32), kGatherWaves);
    p.rows_per_slab = cap_slab_rows(round_up(cdiv(N, want), 32), sizeof(double));
    p.nslab = (int)cdiv(N, p.rows_per_slab);
  } else if (p.wide && N > 0 && K > 0) {
    // About two rounds of pass-2 waves at two waves per SIMD, within the partials' cap.
    int64_t want = cdiv((int64_t)16 * current_device_cus(), K * p.nstrip);
    const int64_t cap = (int64_t)(kWidePartBytes / ((size_t)p.KP * p.NSB * 1024 * sizeof(float)));
    if (want > cap) want = cap;
    if (want > cdiv(N, 32)) want = cdiv(N, 32);
    if (want < 1) want = 1;
    p.rows_per_slab = round_up(cdiv(N, want), 32);
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
  // The bf16 contract's operands: bf16(L) and b in fp32.
  p.off_lop = off;
  if (bf16) off = align256(off + (size_t)p.KP * p.DP * p.DP * sizeof(__bf16));
  p.off_bsw = off;
  if (bf16) off = align256(off + (size_t)p.KP * p.DP * sizeof(float));
  p.off_ck = off;       off = align256(off + (size_t)p.KP * sizeof(double));
  // Split-bf16 operands of pass 1: 4 bf16x8 per (16 dimensions, 32 coordinates, lane).
  const bool x6 = !bf16;
  p.off_l3 = off;
  if (x6) off = align256(off + (size_t)p.KP * (p.DP / 32) * (p.DP / 16) * 4 * 64 * sizeof(bf16x8));
  p.off_esw = off;
  if (x6) off = align256(off + (size_t)p.KP * p.DP * sizeof(double));
  p.off_rowstat = off;  off = align256(off + (size_t)(N > 0 ? N : 0) * sizeof(double));
  p.off_part_sig = off;
  off = align256(off + (size_t)p.npart * p.KP * (bf16 ? p.NMB * p.NMB : p.NSB) * 1024 * sizeof(float));
  p.off_part_mu = off;  off = align256(off + (size_t)p.npart * p.KP * p.DP * sizeof(float));
  p.off_part_nk = off;  off = align256(off + (size_t)p.npart * p.KP * sizeof(float));
  p.off_lj = off;
  if (p.lj || p.keep_lj || p.autolj) off = align256(off + full_lj_bytes(N, p.KP));
  // Need masks: one word per (32-row tile of the pass-1 grid, component).
  p.grid1 = 0;
  p.off_need = off;
  if (p.need) off = align256(off + (size_t)round_up(cdiv(N, 32), 8) * p.KP * sizeof(unsigned));
  p.off_bound = off;
  if (p.need && N > 0) {
    const int tpw = full_x6_tpw(p.DP);
    p.grid1 = (int)std::min<int64_t>(cdiv(N, 32 * kWaves * tpw), (int64_t)full_waves_per_eu(p.DP) * current_device_cus());
    const size_t slot_rows = (size_t)p.grid1 * kWaves * 32 * tpw;
    if (p.needmode == kNeedBounds) off = align256(off + slot_rows * p.KP * sizeof(unsigned short));
    if (p.needmode == kNeedLists) off = align256(off + slot_rows * full_list_spill(p.DP, (int)K) * sizeof(unsigned));
  }
  p.off_probe = off;
  if (p.autolj) off = align256(off + probe_bytes() + (size_t)p.nprobe * p.KP * 32 * sizeof(float));
  p.total = off;
  return p;
}

// ---------------------------------------------------------------------------
// Pass 1 on the bf16 matrix cores: the whitening in the centred
// split-bf16 form of the isotropic pass 1 (x6c_tile, fgmm_common.hpp).  V^T =
// L_k^T X^T over chunks of 16 dimensions; the A operand is L_k^T split exactly into
// three bf16 plus, in a fourth slot, the chunk's centring offsets
// -o_qj = -fp32(sum over d in chunk q of L_k,dj mu_k,d) against a ones operand, so
// each chunk adds L_k[q]^T (x - mu_k)[q] - a small number for the rows near the
// component - to the fp32 accumulator.  The offsets come back in fp64:
// v_j = t_j + e_j with e_j = sum_q o_qj - b_j.  Six of the nine split products are
// kept (the dropped ones are below 2^-24 of the largest), so v carries the error of
// an fp32 contraction of the centred row, not of L^T x against b.
//
//   l3[k][mb][q][s][lane] (bf16x8): s < 3: split s of L_k[16q + 8g + e][32 mb + c];
//                                   s = 3: splits of -o_q,32mb+c in elements 0..2 (g = 0)
//   esw[k][mb][g][i]     (f64):    e_j, j = 32 mb + acc_row(i, g)
// ---------------------------------------------------------------------------

//   ck[k]                (f64):    c_k
// One 256-thread workgroup per component k < KP.
__global__ __launch_bounds__(256) void full_x6_prep(const float* __restrict__ mu, int64_t ldmu,
                                                    const float* __restrict__ L, int64_t K, int D, int DP,
                                                    const float* __restrict__ lpi, bf16x8* __restrict__ l3,
                                                    double* __restrict__ esw, double* __restrict__ ck) {
  __shared__ double so[16][256];  // o_qj, DP <= 256
  __shared__ double se[256];      // e_j, then log |L_jj|
  const int64_t k = blockIdx.x;
  const int tid = threadIdx.x, lane = tid & 63, wave = tid >> 6;
  const int c = lane & 31, g = lane >> 5;
  const bool valid = k < K;
  const float* Lk = L + k * (int64_t)D * D;
  const int NQ = DP / 16, NMB = DP / 32;
  // o_qj = sum over d in chunk q of L_dj mu_d (fp64), one (q, j) per thread.
  for (int idx = tid; idx < NQ * DP; idx += 256) {
    const int q = idx / DP, j = idx % DP;
    double o = 0.0;
    if (valid && j < D)
#pragma unroll 8
      for (int d = 16 * q; d < 16 * q + 16 && d < D; ++d) o = fma((double)Lk[(int64_t)d * D + j], (double)mu[k * ldmu + d], o);
    so[q][j] = o;
  }
  __syncthreads();
  // e_j = sum_q fp32(o_qj) - b_j with b_j = sum_q o_qj, both summed in q order.
  if (tid < DP) {
    double b = 0.0, osum = 0.0;
    for (int q = 0; q < NQ; ++q) {
      osum += (double)(float)so[q][tid];
      b += so[q][tid];
    }
    se[tid] = osum - b;
  }
  __syncthreads();
  // Operands: (mb, q) pairs dealt over the four waves.
  for (int pq = wave; pq < NMB * NQ; pq += 4) {
    const int mb = pq / NQ, q = pq % NQ;
    const int j = 32 * mb + c;
    f32x4 lo = zero4(), hi = zero4();
#pragma unroll
    for (int e = 0; e < 4; ++e) {
      const int d0 = 16 * q + 8 * g + e, d1 = d0 + 4;
      lo[e] = (valid && d0 < D && j < D) ? Lk[(int64_t)d0 * D + j] : 0.0f;
      hi[e] = (valid && d1 < D && j < D) ? Lk[(int64_t)d1 * D + j] : 0.0f;
    }
    bf16x8 sp[3];
    split3_bf16(lo, hi, sp);
    bf16x8* dst = l3 + (((k * NMB + mb) * NQ + q) * 4) * 64 + lane;
#pragma unroll
    for (int t = 0; t < 3; ++t) dst[t * 64] = sp[t];
    // Offset slot: -o_qj in k slots 0..2 (lane-half 0), against x6c_ones.
    const float mo = -(float)so[q][j];
    const f32x4 olo = {g == 0 ? mo : 0.0f, 0.0f, 0.0f, 0.0f};
    bf16x8 os[3];
    split3_bf16(olo, zero4(), os);
    bf16x8 ov;
#pragma unroll
    for (int e = 0; e < 8; ++e) ov[e] = (__bf16)0.0f;
    ov[0] = os[0][0];
    ov[1] = os[1][0];
    ov[2] = os[2][0];
    dst[3 * 64] = ov;
  }
  if (tid < DP) {
    const int mb = tid / 32, gg = (tid >> 4) & 1, i = tid & 15;
    esw[(k * NMB + mb) * 32 + gg * 16 + i] = se[32 * mb + acc_row(i, gg)];
  }
  __syncthreads();
  // c_k, the log-determinant summed in d order.
  if (tid < D) se[tid] = valid ? log(fabs((double)Lk[(int64_t)tid * D + tid]) + 1e-30) : 0.0;
  __syncthreads();
  if (tid == 0) {
    double c0 = -INFINITY;
    if (valid) {
      double ld = 0.0;
      for (int d = 0; d < D; ++d) ld += se[d];
      c0 = ((double)lpi[k] + ld - 0.5 * (double)D * kLog2Pi) * kLog2e;
    }
    ck[k] = c0;
  }
}


// What pass 1 leaves for pass 2 besides logZ2.
constexpr int kLjmStore = 1;   // the stored log-joint
constexpr int kLjmNeed = 2;    // need masks only (the default plan)

// With need masks (LJM == kLjmNeed) the grid is persistent: workgroup b takes the
// tile groups b, b + gridDim.x, ... of 32 kWaves TPW rows (TPW = full_x6_tpw 32-row
// tiles per wave).  Wave w of workgroup b keeps, in its slot 4 b + w of `bound`, the
// workspace part of its rows' candidate lists (needmode kNeedLists, [row][entry]
// words, the first entries in LDS) or the bf16 upper bounds of its rows' log-joint
// (kNeedBounds, [tile][component][row]); each lane reads back its own writes once
// logZ2 is final.  The wave writes the need word of each (32-row tile, component): bit
// r set unless the bound of row r is kLjNeedGap below its logZ2 (need_put_masks).
// KEEP (with need masks): also store the log-joint, for a pass 2 that reads r.  NM is
// the need-mask form (one body per form keeps the others' registers out of the
// contraction loop).
template <int DP, int LJM, bool KEEP = false, int NM = kNeedRunMax>
__global__ __attribute__((amdgpu_flat_work_group_size(kThreads, kThreads),
                          amdgpu_waves_per_eu(full_waves_per_eu(DP), full_waves_per_eu(DP))))
void full_lse_x6(const float* __restrict__ X, int64_t ldx, int64_t N, int D, const bf16x8* __restrict__ l3,
                 const double* __restrict__ esw, const double* __restrict__ ck, int K, int KP,
                 float* __restrict__ logZ, double* __restrict__ rowstat, float* __restrict__ lj,
                 unsigned* __restrict__ need, unsigned short* __restrict__ bound, int dense, ProbeSel probe) {
  constexpr int needmode = NM;
  constexpr bool LJ = LJM == kLjmStore || KEEP;
  static_assert(!KEEP || LJM == kLjmNeed, "KEEP adds the log-joint to the need masks");
  // The stored branch's instance (D <= 64): its pass 2 (full_accum_ljt) reads r from
  // the kept log-joint and no need masks, so none are formed.  Above D = 128 the
  // gathering pass 2 reads both.
  constexpr bool MASKS = LJM == kLjmNeed && !(KEEP && flj_applies(DP));
  // FGMM_FLAG_STORE_LOGJOINT_AUTO launches both need-mask instances; the probe's
  // counts let the KEEP one (the stored branch) or the other run.
  if (probe.count != nullptr && probe_selects(probe) != KEEP) return;
  constexpr int NMB = DP / 32, NQ = DP / 16;
  constexpr int SMB = full_x6_smb(DP);            // coordinate blocks per stage
  constexpr int NST = NMB / SMB;                  // stages per component
  constexpr int BLK = full_x6_stage(DP);          // bf16x8 per stage
  constexpr int LPT = BLK / kThreads;
  constexpr int NE = 32 * SMB;                    // e values per stage
  constexpr int BW = NE + 8;                      // doubles per stage (e, then c)
  constexpr int TPW = full_x6_tpw(DP);            // 32-row tiles per wave
  constexpr int NC = full_list_cands(DP);         // candidates per row in LDS
  static_assert(BLK % kThreads == 0 && kThreads > NE, "even split");

  extern __shared__ __align__(16) unsigned char lds_raw[];
  bf16x8* l_l = reinterpret_cast<bf16x8*>(lds_raw);                                // [2][BLK]
  double* e_l = reinterpret_cast<double*>(lds_raw + 2 * BLK * sizeof(bf16x8));     // [2][BW]

  const int tid = threadIdx.x, lane = tid & 63;
  const int wave = __builtin_amdgcn_readfirstlane(tid >> 6);
  const int c = lane & 31, g = lane >> 5;
  const bool lists = MASKS && needmode == kNeedLists;
  // kNeedLists: the wave's LDS candidates [NC][TPW * 32 rows] (component << 16 | bf16
  // bound), then its mask words [TPW][KP]; the rest of row u's list at spill + u 32 nsp.
  unsigned* cand_l = reinterpret_cast<unsigned*>(lds_raw + full_x6_lds_bytes(DP)) +
                     wave * TPW * (NC * 32 + KP);
  unsigned* word_l = cand_l + NC * 32 * TPW;
  if (lists)
    for (int k = lane; k < TPW * KP; k += 64) word_l[k] = 0u;
  const int nsp = full_list_spill(DP, K);
  const int64_t slot = (int64_t)blockIdx.x * kWaves + wave;
  unsigned* spill = lists ? reinterpret_cast<unsigned*>(bound) + (slot * TPW * 32 + c) * nsp : nullptr;
  unsigned short* bnd = MASKS && needmode == kNeedBounds ? bound + slot * TPW * 32 * KP : nullptr;
  const int64_t ntw = cdiv(N, 32 * kWaves * TPW);
  const int64_t tw_step = LJM == kLjmNeed ? (int64_t)gridDim.x : ntw;

  for (int64_t tw = blockIdx.x; tw < ntw; tw += tw_step) {
  int64_t tile[TPW];   // the wave's 32-row tiles
  bool valid[TPW];     // this lane's row of each
  int ncand[TPW];      // the row's listed candidates (kNeedLists; lanes of half-wave 0)
#pragma unroll
  for (int u = 0; u < TPW; ++u) {
    tile[u] = (tw * kWaves + wave) * TPW + u;
    valid[u] = tile[u] * 32 + c < N;
    ncand[u] = 0;
  }

  // Stage s = k NST + sub holds blocks SMB sub .. of component k: contiguous in l3
  // and esw.  Both reach LDS buffer s & 1 by buffer-to-LDS loads (no staging
  // registers): LPT 16-byte pieces per lane of the operands, and the NE e values from
  // the first NE / 2 lanes of wave 0.
  auto fetch = [&](int64_t s) {
    const DmaSrc r = dma_src(l3 + s * BLK, (uint32_t)(BLK * sizeof(bf16x8)));
    bf16x8* dst = l_l + (s & 1) * BLK + wave * 64;
#pragma unroll
    for (int q = 0; q < LPT; ++q)
      lds_dma16(r, dst + q * kThreads, tid * (int)sizeof(bf16x8), q * kThreads * (int)sizeof(bf16x8));
    if (wave == 0 && lane < NE / 2) {
      const DmaSrc re = dma_src(esw + s * NE, (uint32_t)(NE * sizeof(double)));
      lds_dma16(re, e_l + (s & 1) * BW, lane * 16, 0);
    }
  };
  fetch(0);
  // This lane's rows, dimensions 16q + 8g .. +7, split three ways.
  bf16x8 xb[TPW][NQ][3];
#pragma unroll
  for (int u = 0; u < TPW; ++u) {
    const int64_t row = tile[u] * 32 + c;
#pragma unroll
    for (int q = 0; q < NQ; ++q) {
      const int d0 = 16 * q + 8 * g;
      split3_bf16(load_row4(X, ldx, row, d0, D, valid[u]), load_row4(X, ldx, row, d0 + 4, D, valid[u]),
                  xb[u][q]);
    }
  }
  const bf16x8 ones = x6c_ones(lane);
  dma_barrier();

  const double hl = 0.5 * kLog2e;
  double mx[TPW], maha[TPW];
  float sm[TPW], run_max[TPW];   // run_max: the running-max need bound (not kNeedBounds)
#pragma unroll
  for (int u = 0; u < TPW; ++u) {
    mx[u] = -INFINITY;
    maha[u] = 0.0;
    sm[u] = 0.0f;
    run_max[u] = -INFINITY;
  }
  const int64_t nstage = (int64_t)K * NST;
  for (int64_t s = 0; s < nstage; ++s) {
    const int buf = (int)(s & 1);
    if (s + 1 < nstage) fetch(s + 1);
    // Component s / NST completes with this stage: its constant, read early.
    const bool done = NST == 1 || (int)(s % NST) == NST - 1;
    const double ckv = done ? ck[s / NST] : 0.0;
    const bf16x8* lc = l_l + buf * BLK + lane;
    const double* ec = e_l + buf * BW;
#pragma unroll
    for (int mb = 0; mb < SMB; ++mb) {
      // lane = row, register i = whitened coordinate 32 mb + acc_row(i, g).  One
      // accumulation chain per tile: no chain sums, and 3.12 ms against 3.56 ms with
      // four at N=250K, K=256, D=64.
      f32x16 t[TPW];
      x6c_tile_multi<NQ, TPW>([&](int q, int v) { return lc[((mb * NQ + q) * 4 + v) * 64]; }, xb, ones, t);
      const double* eb = ec + mb * 32 + g * 16;
#pragma unroll
      for (int i = 0; i < 16; ++i) {
        const double e = eb[i];
#pragma unroll
        for (int u = 0; u < TPW; ++u) {
          const double v = (double)t[u][i] + e;
          maha[u] = fma(v, v, maha[u]);
        }
      }
    }
    // Stage s + 1 has landed and every wave is done with buffer buf, which stage s + 2
    // fills; what follows reads registers only.  The stores below are in flight behind
    // the next stage's contraction (this wait also drains them, a stage later).
    dma_barrier();
    if (done) {   // component s / NST complete
      const int k = (int)(s / NST);
#pragma unroll
      for (int u = 0; u < TPW; ++u) {
        maha[u] += __shfl_xor(maha[u], 32);
        const double ll = ckv - hl * maha[u];
        // Both half-waves hold row c's log-joint; both store it (same value, address).
        if constexpr (LJ) lj[(tile[u] * KP + k) * 32 + c] = (float)ll;
        if constexpr (MASKS) {
          if (needmode == kNeedBounds) {
            if (g == 0) bnd[((int64_t)u * KP + k) * 32 + c] = bf16_bits_up((float)ll);
          } else {
            // logZ2 >= the row's final maximum >= run_max (less a rounding), so a
            // component kLjSkipGap below the running max cannot reach need_put_masks'
            // test (with |run_max| < 2^24, where those roundings stay far inside the
            // margin).
            run_max[u] = fmaxf(run_max[u], (float)ll);
            const bool near = !(fabsf(run_max[u]) < 0x1p24f && (float)ll - run_max[u] < -kLjSkipGap);
            if (lists) {
              // A candidate goes on the row's list (the LDS part, then the workspace
              // part), or past its end sets its bit now.
              if (valid[u] && g == 0 && dense == 0 && near) {
                const unsigned e = ((unsigned)k << 16) | bf16_bits_up((float)ll);
                const int n = ncand[u];
                if (n < NC) {
                  cand_l[n * TPW * 32 + u * 32 + c] = e;
                  ncand[u] = n + 1;
                } else if (n < NC + nsp) {
                  spill[(int64_t)u * 32 * nsp + n - NC] = e;
                  ncand[u] = n + 1;
                } else {
                  atomicOr(word_l + u * KP + k, 1u << c);
                }
              }
            } else {
              const unsigned bits = (unsigned)__builtin_amdgcn_ballot_w64(valid[u] && (dense != 0 || near));
              if (lane == 0) need[tile[u] * KP + k] = bits;
            }
          }
        }
        const double mn = fmax(mx[u], ll);
        const double ms = (mn == -INFINITY) ? 0.0 : mn;
        sm[u] = sm[u] * fast_exp2((float)(mx[u] - ms)) + fast_exp2((float)(ll - ms));
        mx[u] = mn;
        maha[u] = 0.0;
      }
    }
  }
#pragma unroll
  for (int u = 0; u < TPW; ++u) {
    const int64_t row = tile[u] * 32 + c;
    const double lz2 = mx[u] + (double)log2f(sm[u]);
    if (valid[u] && g == 0) {
      rowstat[row] = lz2;
      if (logZ) logZ[row] = (float)(lz2 * kLn2);
    }
    if constexpr (MASKS) {
      if (needmode == kNeedBounds) {
        const unsigned short* bt = bnd + (int64_t)u * KP * 32 + c;
        if (g == 0)
          need_put_masks([&](int k) { return bf16_bits_to_float(bt[(int64_t)k * 32]); }, need + tile[u] * KP,
                         nullptr, K, c, lz2, valid[u], dense != 0);
      } else if (lists) {
        // need_put_masks' test on the row's candidates, then the words out (coalesced)
        // and cleared for the next tile.  A row whose logZ2 is NaN gets every bit, and
        // with `dense` every valid row does, as need_put_masks gives them.
        const float zx = (float)lz2;
        const float zy = (lz2 > -INFINITY && lz2 < INFINITY) ? (float)(lz2 - (double)zx) : 0.0f;
        unsigned* wu = word_l + u * KP;
        for (int i = 0; i < ncand[u]; ++i) {
          const unsigned e = i < NC ? cand_l[i * TPW * 32 + u * 32 + c] : spill[(int64_t)u * 32 * nsp + i - NC];
          const float R = bf16_bits_to_float((unsigned short)(e & 0xffffu));
          if (!(((R - zx) - zy) < -kLjNeedGap)) atomicOr(wu + (e >> 16), 1u << c);
        }
        const unsigned vbits = (unsigned)__builtin_amdgcn_ballot_w64(valid[u] && g == 0);
        const unsigned nanbits = (unsigned)__builtin_amdgcn_ballot_w64(valid[u] && g == 0 && lz2 != lz2);
        asm volatile("s_waitcnt lgkmcnt(0)" ::: "memory");   // the wave's ORs before its reads
        for (int k = lane; k < K; k += 64) {
          need[tile[u] * KP + k] = dense != 0 ? vbits : (wu[k] | nanbits);
          wu[k] = 0u;
        }
      } else {
        // A row whose logZ2 is NaN gets its bit for every component, as the exact test
        // gives it.
        const unsigned nanbits = (unsigned)__builtin_amdgcn_ballot_w64(valid[u] && g == 0 && lz2 != lz2);
        if (lane == 0 && nanbits != 0)
          for (int k = 0; k < K; ++k) need[tile[u] * KP + k] |= nanbits;
      }
    }
  }
  }
}

// ---------------------------------------------------------------------------
// The probe of FGMM_FLAG_STORE_LOGJOINT_AUTO (D <= 64, K <= kProbeMaxKB), in two
// kernels.  full_probe_ll: kProbeSplit workgroups per sampled 32-row tile, each over
// a quarter of the components, form the rows' log-joint from the whitening's
// centring step and x1 L1 product only (an error of a few log2 units against the
// kLjNeedGap = 160 margin) into `lls` ([tile][KP][32] floats).  full_probe_count:
// per row, the components with ll >= M - kLjNeedGap (M the row's largest) are
// counted, an estimate of the pairs pass 1 marks as needed; the tile's count is
// written, and the kernels that need the choice sum the counts (probe_selects).
// ---------------------------------------------------------------------------
constexpr int kProbeWaves = 16;
constexpr int kProbeSplit = 4;
template <int DP>
__global__ __launch_bounds__(64 * kProbeWaves) void full_probe_ll(const float* __restrict__ X, int64_t ldx,
                                                                  int64_t N, int D,
                                                                  const bf16x8* __restrict__ l3,
                                                                  const double* __restrict__ esw,
                                                                  const double* __restrict__ ck, int K, int KP,
                                                                  int ntile, float* __restrict__ lls) {
  constexpr int NMB = DP / 32, NQ = DP / 16;
  const int s = blockIdx.x / kProbeSplit, part = blockIdx.x % kProbeSplit;
  const int tid = threadIdx.x, lane = tid & 63;
  const int wave = __builtin_amdgcn_readfirstlane(tid >> 6);
  const int c = lane & 31, g = lane >> 5;
  const int64_t tile = probe_tile(s, N, ntile);
  const int64_t row = tile * 32 + c;
  const bool valid = row < N;

  bf16x8 xh[NQ];
#pragma unroll
  for (int q = 0; q < NQ; ++q) {
    const int d0 = 16 * q + 8 * g;
    xh[q] = to_bf16x8(load_row4(X, ldx, row, d0, D, valid), load_row4(X, ldx, row, d0 + 4, D, valid));
  }
  const bf16x8 ones = x6c_ones(lane);
  const double hl = 0.5 * kLog2e;
  for (int k = part * kProbeWaves + wave; k < K; k += kProbeSplit * kProbeWaves) {
    double maha = 0.0;
#pragma unroll
    for (int mb = 0; mb < NMB; ++mb) {
      const bf16x8* lp = l3 + ((int64_t)k * NMB + mb) * NQ * 4 * 64 + lane;
      f32x16 acc[2] = {zero16(), zero16()};
#pragma unroll
      for (int q = 0; q < NQ; ++q) {
        acc[q & 1] = mfma_bf16(lp[(q * 4 + 3) * 64], ones, acc[q & 1]);
        acc[q & 1] = mfma_bf16(lp[(q * 4 + 0) * 64], xh[q], acc[q & 1]);
      }
      const double* eb = esw + ((int64_t)k * NMB + mb) * 32 + g * 16;
#pragma unroll
      for (int i = 0; i < 16; ++i) {
        const double v = (double)(acc[0][i] + acc[1][i]) + eb[i];
        maha = fma(v, v, maha);
      }
    }
    maha += __shfl_xor(maha, 32);
    if (g == 0) lls[((int64_t)s * KP + k) * 32 + c] = (float)(ck[k] - hl * maha);
  }
}

__global__ __launch_bounds__(256) void full_probe_count(int64_t N, int K, int KP, int ntile,
                                                        const float* __restrict__ lls,
                                                        unsigned* __restrict__ count) {
  __shared__ float mrow[8][32];
  __shared__ unsigned part[4];
  const int s = blockIdx.x;
  const int tid = threadIdx.x, lane = tid & 63, wave = tid >> 6;
  const int c = tid & 31, grp = tid >> 5;   // 8 groups of 32 lanes, each over every 8th component
  const int64_t tile = probe_tile(s, N, ntile);
  const bool valid = tile * 32 + c < N;
  const float* lt = lls + (int64_t)s * KP * 32 + c;
  float M = -INFINITY;
  for (int k = grp; k < K; k += 8) M = fmaxf(M, lt[k * 32]);
  mrow[grp][c] = M;
  __syncthreads();
  M = mrow[0][c];
#pragma unroll
  for (int j = 1; j < 8; ++j) M = fmaxf(M, mrow[j][c]);
  unsigned need = 0;
  if (valid)
    for (int k = grp; k < K; k += 8) need += (lt[k * 32] - M >= -kLjNeedGap) ? 1u : 0u;
#pragma unroll
  for (int o = 32; o > 0; o >>= 1) need += __shfl_xor(need, o);
  if (lane == 0) part[wave] = need;
  __syncthreads();
  if (tid == 0) count[s] = part[0] + part[1] + part[2] + part[3];
}

// ---------------------------------------------------------------------------
// Pass 2 of the stored plan (FGMM_FLAG_STORE_LOGJOINT): r from the log-joint pass 1
// stored, no whitening.
// ---------------------------------------------------------------------------
template <int DP>
constexpr size_t accum_lds_bytes() {
  constexpr int TR = 32 * kRowGroups;
  return (size_t)2 * TR * (DP + 4) * sizeof(float)              // X tiles
         + (size_t)2 * TR * sizeof(double)                      // logZ2
         + (size_t)kAccWaves * 32 * sizeof(float);              // r exchange
}

template <int DP>
__global__ __attribute__((amdgpu_flat_work_group_size(kAccThreads, kAccThreads), amdgpu_waves_per_eu(2, 2)))
void full_accum(const float* __restrict__ X, int64_t ldx, int64_t N, int D, int K, int KP,
                const double* __restrict__ rowstat, int nslab, int64_t rows_per_slab,
                float* __restrict__ part_sig, float* __restrict__ part_mu, float* __restrict__ part_nk,
                int dense, const float* __restrict__ lj) {
  constexpr int NMB = DP / 32, NSB = NMB * (NMB + 1) / 2;
  constexpr int RS = DP + 4, V4 = DP / 4;
  constexpr int TR = 32 * kRowGroups;
  constexpr int LPT = (TR * V4) / kAccThreads;
  static_assert((TR * V4) % kAccThreads == 0, "even split");

  extern __shared__ __align__(16) unsigned char lds_raw[];
  unsigned char* p = lds_raw;
  float* xs = reinterpret_cast<float*>(p);    p += 2 * TR * RS * sizeof(float);
  double* rs = reinterpret_cast<double*>(p);  p += 2 * TR * sizeof(double);
  float* r_l = reinterpret_cast<float*>(p);

  const int tid = threadIdx.x, lane = tid & 63, wave = tid >> 6;
  const int c = lane & 31, g = lane >> 5;
  const int cw = wave & 3, rg = wave >> 2;
  const int slab = blockIdx.x % nslab;
  const int cg = blockIdx.x / nslab;
  const int k = cg * kCompsPerWG + cw;
  const bool active = k < K;

  const int64_t r_begin = (int64_t)slab * rows_per_slab;
  int64_t r_end = r_begin + rows_per_slab;
  if (r_end > N) r_end = N;
  const int ntiles = r_end > r_begin ? (int)cdiv(r_end - r_begin, TR) : 0;

  f32x16 acc[NSB];
#pragma unroll
  for (int s = 0; s < NSB; ++s) acc[s] = zero16();
  float mua[NMB];
#pragma unroll
  for (int mb = 0; mb < NMB; ++mb) mua[mb] = 0.0f;
  float nk = 0.0f;

  f32x4 stage[LPT];
  double rstage = INFINITY;
  const bool full_d = (D == DP);
  auto fetch = [&](int t) {
    const int64_t row0 = r_begin + (int64_t)t * TR;
    if (full_d && row0 + TR <= r_end) {
      // Interior tile: no row or column masking.
      const float* src = X + row0 * ldx;
#pragma unroll
      for (int q = 0; q < LPT; ++q) {
        const int idx = q * kAccThreads + tid;
        stage[q] = *reinterpret_cast<const f32x4*>(src + (int64_t)(idx / V4) * ldx + (idx % V4) * 4);
      }
    } else {
#pragma unroll
      for (int q = 0; q < LPT; ++q) {
        const int idx = q * kAccThreads + tid;
        const int rr = idx / V4, c4 = idx % V4;
        const int64_t row = row0 + rr;
        stage[q] = load_row4(X, ldx, row, c4 * 4, D, row < r_end);
      }
    }
    if (tid < TR) {
      const int64_t row = row0 + tid;
      rstage = (row < r_end) ? rowstat[row] : INFINITY;
    }
  };
  auto commit = [&](int buf) {
    float* dst = xs + buf * TR * RS;
#pragma unroll
    for (int q = 0; q < LPT; ++q) {
      const int idx = q * kAccThreads + tid;
      const int rr = idx / V4, c4 = idx % V4;
      *reinterpret_cast<f32x4*>(dst + rr * RS + c4 * 4) = stage[q];
    }
    if (tid < TR) rs[buf * TR + tid] = rstage;
  };

  // The stored log-joint of this wave's component for row c of tile t (0 past the
  // slab, where logZ2 = +inf makes r = 0), loaded one tile ahead where the register
  // fits (at D = 128 the accumulators leave none).
  constexpr bool PF = DP <= 96;
  auto lj_of = [&](int t) -> float {
    const int64_t row0 = r_begin + (int64_t)t * TR + rg * 32;
    return (active && row0 < r_end) ? lj[((row0 >> 5) * KP + k) * 32 + c] : 0.0f;
  };
  float lnext = 0.0f;
  if (ntiles > 0) {
    fetch(0);
    if (PF) lnext = lj_of(0);
    commit(0);
  }
  __syncthreads();

  float* rx = r_l + wave * 32;
  for (int t = 0; t < ntiles; ++t) {
    const int buf = t & 1;
    const bool more = t + 1 < ntiles;
    const float* xt = xs + buf * TR * RS + rg * 32 * RS;
    const double* rt = rs + buf * TR + rg * 32;
    const float l = PF ? lnext : lj_of(t);
    if (PF && more) lnext = lj_of(t + 1);
    float rv = 0.0f;
    if (active) {
      // r for this lane's row c (both half-waves hold it).
      rv = fast_exp2((float)((double)l - rt[c]));
      if (g == 0) {
        nk += rv;
        rx[c] = rv;
      }
    }
    if (more) fetch(t + 1);
    __builtin_amdgcn_wave_barrier();
    if (active) {
      // sig_outer[d1][d2] += sum_rows (r x_d1) x_d2 over the tile's 32 rows.  Step s
      // takes rows r0 + 4g (r0 = 8 (s >> 2) + (s & 3)) for half g, matching the
      // A-operand k index of each half-wave; a step whose two rows have zero
      // responsibility adds nothing, so the loop visits the steps with a nonzero row
      // (bit r0 of the pair mask), in ascending order.
      const unsigned nz = (unsigned)__builtin_amdgcn_ballot_w64(rv != 0.0f);   // lanes 0..31: rows
      unsigned pm = dense ? 0x0f0f0f0fu : lj_pair_mask(nz);
      while (pm != 0u) {
        const int r0 = __builtin_ctz(pm);
        pm &= pm - 1u;
        const int row = r0 + 4 * g;
        const float rr = rx[row];
        float xv[NMB], av[NMB];
#pragma unroll
        for (int mb = 0; mb < NMB; ++mb) {
          xv[mb] = xt[row * RS + 32 * mb + c];
          av[mb] = rr * xv[mb];
          mua[mb] += av[mb];
        }
        int sb = 0;
#pragma unroll
        for (int m1 = 0; m1 < NMB; ++m1) {
#pragma unroll
          for (int m2 = m1; m2 < NMB; ++m2) {
            acc[sb] = mfma32(av[m1], xv[m2], acc[sb]);
            ++sb;
          }
        }
      }
    }
    if (more) commit(buf ^ 1);
    __syncthreads();
  }

  if (active) {
    const int64_t pbase = ((int64_t)slab * kRowGroups + rg) * KP + k;
    float* ps = part_sig + pbase * NSB * 1024;
#pragma unroll
    for (int sb = 0; sb < NSB; ++sb) {
#pragma unroll
      for (int i = 0; i < 16; ++i) ps[sb * 1024 + acc_row(i, g) * 32 + c] = acc[sb][i];
    }
#pragma unroll
    for (int mb = 0; mb < NMB; ++mb) {
      const float v = mua[mb] + __shfl_xor(mua[mb], 32);
      if (g == 0) part_mu[pbase * DP + 32 * mb + c] = v;
    }
    float nks = nk;
#pragma unroll
    for (int o = 16; o >= 1; o >>= 1) nks += __shfl_xor(nks, o);
    if (lane == 0) part_nk[pbase] = nks;
  }
}

// Finish of mu_acc and Nk: one thread per (k, d) of mu_acc and per k of Nk.
// ATOMIC (FGMM_FLAG_ATOMIC_REDUCE): partial blockIdx.y is added with float atomics into
// the zeroed (or accumulated) outputs instead of the fixed-order fp64 sum.
template <bool ATOMIC>
__global__ __launch_bounds__(256) void full_reduce(const float* __restrict__ part_mu,
                                                   const float* __restrict__ part_nk, int npart, int KP,
                                                   int DP, int64_t K, int D,
                                                   float* __restrict__ Nk, float* __restrict__ mu_acc,
                                                   int accumulate) {
  // Sum over the partials of p[0], p[stride], ... (or, atomically, the one of this grid row).
  auto finish = [&](const float* p, int64_t stride, float* o) {
    if (ATOMIC) {
      atomicAdd(o, p[(int64_t)blockIdx.y * stride]);
    } else {
      const double s = strided_sum(p, npart, stride);
      *o = accumulate ? (float)((double)*o + s) : (float)s;
    }
  };
  const int64_t j = (int64_t)blockIdx.x * blockDim.x + threadIdx.x;
  if (j < K * D) {
    const int64_t k = j / D;
    const int d = (int)(j % D);
    finish(part_mu + k * DP + d, (int64_t)KP * DP, mu_acc + j);
    return;
  }
  const int64_t kk = j - K * D;
  if (kk < K) finish(part_nk + kk, KP, Nk + kk);
}

// sig_outer: one workgroup per (component k, upper 32x32 block sb = (b1, b2)).  The
// block's partials are read coalesced and summed in partial order in fp64 (or, with
// ATOMIC, partial blockIdx.y alone is taken); the sums go through LDS so that both the
// (b1, b2) tile and its mirror (b2, b1) are written row-contiguously.  A diagonal
// block's upper triangle is mirrored onto its lower one, so sig_outer is exactly
// symmetric.
template <bool ATOMIC>
__global__ __launch_bounds__(256) void full_reduce_sig(const float* __restrict__ part_sig, int npart, int KP,
                                                       int NMB, int D, float* __restrict__ sig_outer,
                                                       int accumulate) {
  __shared__ double tile[32][33];
  const int NSB = NMB * (NMB + 1) / 2;
  const int k = (int)(blockIdx.x / NSB);
  const int sb = (int)(blockIdx.x % NSB);
  int b1 = 0, rem = sb;
  while (rem >= NMB - b1) {
    rem -= NMB - b1;
    ++b1;
  }
  const int b2 = b1 + rem;
  const int tid = threadIdx.x;
  const int64_t pstride = (int64_t)KP * NSB * 1024;
  const float* p = part_sig + ((int64_t)k * NSB + sb) * 1024;
#pragma unroll
  for (int j = 0; j < 4; ++j) {
    const int e = tid + 256 * j;
    tile[e >> 5][e & 31] = ATOMIC ? (double)p[(int64_t)blockIdx.y * pstride + e] : strided_sum(p + e, npart, pstride);
  }
  __syncthreads();
  float* out = sig_outer + (int64_t)k * D * D;
  auto put = [&](int d1, int d2, double v) {
    float* o = out + (int64_t)d1 * D + d2;
    if (ATOMIC) atomicAdd(o, (float)v);
    else *o = accumulate ? (float)((double)*o + v) : (float)v;
  };
#pragma unroll
  for (int j = 0; j < 4; ++j) {
    const int e = tid + 256 * j;
    const int r = e >> 5, c = e & 31;
    const int d1 = 32 * b1 + r, d2 = 32 * b2 + c;
    if (d1 < D && d2 < D) put(d1, d2, b1 == b2 && r > c ? tile[c][r] : tile[r][c]);
    if (b1 != b2) {
      const int m1 = 32 * b2 + r, m2 = 32 * b1 + c;
      if (m1 < D && m2 < D) put(m1, m2, tile[c][r]);
    }
  }
}

__global__ __launch_bounds__(256) void full_fill(float* __restrict__ p, int64_t n, float v) {
  const int64_t i = (int64_t)blockIdx.x * blockDim.x + threadIdx.x;
  if (i < n) p[i] = v;
}

// ---------------------------------------------------------------------------
// Pass 2 of the default plan: the whitening is recomputed only for the
// (row, component) pairs whose need bit pass 1 set.  One wave per (row slab,
// component); a workgroup holds 4 waves of one component on consecutive slabs,
// with the component's split-bf16 operands (pass 1's l3, esw and c) in LDS.  Each
// wave walks its slab's need words for the component and queues the needed rows;
// per tile of 32 queued rows it stages the rows of X in its LDS tile, whitens them
// as pass 1 does (x6c_tile over the coordinate blocks, the same operands and order,
// so maha and the log-joint are pass 1's), forms r = 2^(ll2 - logZ2), and then
// accumulates Nk, mu_acc and the upper 32x32 blocks of sig_outer = sum r x x^T
// (r-scaled rows as the A operand of six split-bf16 products per 16 rows, only the
// 16-row steps with a nonzero row).  Workgroups are dealt to the 8 XCDs by gather_item: the
// components of a slab group share an XCD's L2 for the rows of X where there are 8
// or more groups, and split over the XCDs that share a group where there are fewer.
// Above D = 128 the upper
// blocks are dealt to gather_sig_groups(DP) launches, GRP = 0, 1, ..., each
// accumulating a contiguous run of blocks (GRP 0 also mu_acc and Nk) after the same
// whitening.
// ---------------------------------------------------------------------------

// Up to D = 96 the component's operands (32 KB at D = 64, 72 KB at 96) sit in LDS;
// at D = 128 (128 KB) they are read from the workspace (L2) by each wave.  Above
// D = 64 the kernel runs one wave per SIMD.
__host__ __device__ constexpr bool gather_ops_in_lds(int DP) { return DP <= 96; }
__host__ __device__ constexpr int gather_waves_per_eu(int DP) { return DP <= 64 ? 2 : 1; }

template <int DP>
constexpr size_t gather_lds_bytes() {
  return (gather_ops_in_lds(DP) ? (size_t)(DP / 32) * (DP / 16) * 4 * 64 * sizeof(bf16x8) : 0)   // operands
         + (size_t)(DP + 8) * sizeof(double)                        // e, then c
         + (size_t)kGatherWaves * 32 * (DP + 4) * sizeof(float)     // X tile per wave
         + (size_t)kGatherWaves * 32 * sizeof(float)                 // r per wave
         + (size_t)kGatherWaves * 64 * sizeof(int);                  // row queue per wave
}
__host__ __device__ constexpr int gather_groups(int nslab) { return (nslab + kGatherWaves - 1) / kGatherWaves; }
__host__ inline int64_t gather_grid(int nslab, int K) { return gather_item_grid(gather_groups(nslab), K); }

// LJR: r comes from the log-joint pass 1 stored (keep_lj plans) instead of a
// whitening of the queued rows.
template <int DP, int GRP, bool LJR = false>
__global__ __attribute__((amdgpu_flat_work_group_size(64 * kGatherWaves, 64 * kGatherWaves),
                          amdgpu_waves_per_eu(gather_waves_per_eu(DP), gather_waves_per_eu(DP))))
void full_accum_gather(const float* __restrict__ X, int64_t ldx, int64_t N, int D,
                       const bf16x8* __restrict__ l3, const double* __restrict__ esw,
                       const double* __restrict__ ck, int K, int KP, const double* __restrict__ rowstat,
                       const unsigned* __restrict__ need, int nslab, int64_t rows_per_slab,
                       float* __restrict__ part_sig, float* __restrict__ part_mu, float* __restrict__ part_nk,
                       int dense, const float* __restrict__ lj, ProbeSel sel) {
  constexpr int NMB = DP / 32, NQ = DP / 16, NSB = NMB * (NMB + 1) / 2;
  constexpr int NGRP = gather_sig_groups(DP);
  if (probe_selects(sel)) return;   // the stored branch's full_accum_ljt takes the call
  constexpr int NSBG = (NSB + NGRP - 1) / NGRP;              // blocks per group
  constexpr int SB0 = GRP * NSBG;                            // this group's blocks SB0 .. SB1 - 1
  constexpr int SB1 = SB0 + NSBG < NSB ? SB0 + NSBG : NSB;
  constexpr bool FIRST = GRP == 0;                           // also mu_acc and Nk
  static_assert(GRP < NGRP && SB0 < NSB, "group of sig blocks");
  constexpr int RS = DP + 4;
  constexpr int BLK = NMB * NQ * 4 * 64;   // bf16x8 per component
  constexpr bool OPS_LDS = gather_ops_in_lds(DP);

  extern __shared__ __align__(16) unsigned char lds_raw[];
  unsigned char* lp = lds_raw;
  bf16x8* l_l = reinterpret_cast<bf16x8*>(lp);   lp += OPS_LDS ? (size_t)BLK * sizeof(bf16x8) : 0;
  double* e_l = reinterpret_cast<double*>(lp);   lp += (size_t)(DP + 8) * sizeof(double);
  float* xt_all = reinterpret_cast<float*>(lp);  lp += (size_t)kGatherWaves * 32 * RS * sizeof(float);
  float* r_all = reinterpret_cast<float*>(lp);   lp += (size_t)kGatherWaves * 32 * sizeof(float);
  int* q_all = reinterpret_cast<int*>(lp);

  const int tid = threadIdx.x, lane = tid & 63;
  const int wave = __builtin_amdgcn_readfirstlane(tid >> 6);
  const int c = lane & 31, g = lane >> 5;
  int sg, k;
  if (!gather_item(blockIdx.x, gather_groups(nslab), K, sg, k)) return;   // uniform over the workgroup
  if constexpr (OPS_LDS && !LJR)
    for (int idx = tid; idx < BLK; idx += 64 * kGatherWaves) l_l[idx] = l3[(int64_t)k * BLK + idx];
  if constexpr (!LJR)
    for (int idx = tid; idx <= DP; idx += 64 * kGatherWaves) e_l[idx] = idx < DP ? esw[(int64_t)k * DP + idx] : ck[k];
  const bf16x8* lops = OPS_LDS ? l_l : l3 + (int64_t)k * BLK;
  __syncthreads();
  const int slab = sg * kGatherWaves + wave;
  if (slab >= nslab) return;   // no barrier follows

  float* xt = xt_all + wave * 32 * RS;
  float* rx = r_all + wave * 32;
  int* q_l = q_all + wave * 64;

  const int64_t r_begin = (int64_t)slab * rows_per_slab;
  int64_t r_end = r_begin + rows_per_slab;
  if (r_end > N) r_end = N;
  const int64_t t_begin = r_begin / 32, t_end = cdiv(r_end, 32);

  auto words = [&](int64_t tb) -> unsigned {
    const int64_t t = tb + lane;
    return t < t_end ? need[t * KP + k] : 0u;
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

  // The tile in flight: lane (c, g) holds row c's dimensions 16q + 8g .. +7.  The rows
  // come through resources over the slab (a lane without a row reads zeros and makes
  // no access, so the loads issue back to back): X so while D fills whole chunks and
  // the slab spans under 2 GiB (uniform), else load_row4.
  f32x4 raw[2 * NQ];
  double rst;
  float lraw = 0.0f;   // LJR: the stored log-joint of the lane's queued row
  const int64_t slab_bytes = (r_end - r_begin) * ldx * (int64_t)sizeof(float);
  const bool xbuf = D == DP && slab_bytes <= ((int64_t)1 << 31) - 256;
  const buf_rsrc xres = make_rsrc(X + r_begin * ldx, xbuf ? (uint32_t)slab_bytes : 0u);
  const buf_rsrc rres = make_rsrc(rowstat + r_begin, (uint32_t)((r_end - r_begin) * sizeof(double)));
  auto issue = [&](int e) {
    const bool ok = e >= 0;
    if (xbuf) {
      const int off = buf_off(ok ? (int)((int64_t)e * ldx * (int64_t)sizeof(float)) + 32 * g : kBufOob);
#pragma unroll
      for (int q = 0; q < NQ; ++q) {
        raw[2 * q] = __builtin_bit_cast(f32x4, __builtin_amdgcn_raw_buffer_load_b128(xres, off, 64 * q, 0));
        raw[2 * q + 1] = __builtin_bit_cast(f32x4, __builtin_amdgcn_raw_buffer_load_b128(xres, off, 64 * q + 16, 0));
      }
    } else {
      const int64_t row = r_begin + (ok ? e : 0);
#pragma unroll
      for (int q = 0; q < NQ; ++q) {
        raw[2 * q] = load_row4(X, ldx, row, 16 * q + 8 * g, D, ok);
        raw[2 * q + 1] = load_row4(X, ldx, row, 16 * q + 8 * g + 4, D, ok);
      }
    }
    const double z = buf_load_f64(rres, buf_off(ok ? e * (int)sizeof(double) : kBufOob));
    rst = ok ? z : INFINITY;
    if constexpr (LJR) {
      const int64_t rr = r_begin + (ok ? e : 0);   // a row of the slab: no branch
      lraw = lj[((rr >> 5) * KP + k) * 32 + (rr & 31)];
    }
  };

  f32x16 acc[SB1 - SB0];
#pragma unroll
  for (int sb = 0; sb < SB1 - SB0; ++sb) acc[sb] = zero16();
  float mua[NMB];
#pragma unroll
  for (int mb = 0; mb < NMB; ++mb) mua[mb] = 0.0f;
  float nk = 0.0f;
  const bf16x8 ones = x6c_ones(lane);
  const double hl = 0.5 * kLog2e;

  // Up to D = 64 the next tile's rows are loaded while a tile is computed; above,
  // the registers they would take are needed by sig_outer's accumulators.
  constexpr bool PREFETCH = DP <= 64;
  int e;
  int cnt = take(e);
  if (PREFETCH && cnt > 0) issue(e);
  while (cnt > 0) {
    if (!PREFETCH) issue(e);
    asm volatile("s_waitcnt lgkmcnt(0)" ::: "memory");   // the previous tile's LDS reads are done
    // Each chunk to the LDS tile, then split three ways (its fp32 registers free after).
    bf16x8 xb[LJR ? 1 : NQ][3];
#pragma unroll
    for (int q = 0; q < NQ; ++q) {
      *reinterpret_cast<f32x4*>(xt + c * RS + 16 * q + 8 * g) = raw[2 * q];
      *reinterpret_cast<f32x4*>(xt + c * RS + 16 * q + 8 * g + 4) = raw[2 * q + 1];
      if constexpr (!LJR) split3_bf16(raw[2 * q], raw[2 * q + 1], xb[q]);
    }
    const double lz2 = rst;
    const float lcur = lraw;
    int en = -1;
    int cnt_next = 0;
    if (PREFETCH) {
      cnt_next = take(en);
      if (cnt_next > 0) issue(en);
    }

    float rv;
    if constexpr (LJR) {
      rv = fast_exp2((float)((double)lcur - lz2));   // r from the stored log-joint
    } else {
      // maha of row c as pass 1 forms it (lane = row, register = coordinate).
      double maha = 0.0;
#pragma unroll DP <= 64 ? NMB : 1
      for (int mb = 0; mb < NMB; ++mb) {
        const f32x16 t = x6c_tile<NQ, 1>([&](int q, int u) { return lops[((mb * NQ + q) * 4 + u) * 64 + lane]; },
                                         xb, ones);
        const double* eb = e_l + mb * 32 + g * 16;
#pragma unroll
        for (int i = 0; i < 16; ++i) {
          const double v = (double)t[i] + eb[i];
          maha = fma(v, v, maha);
        }
      }
      maha += __shfl_xor(maha, 32);
      const double ll = e_l[DP] - hl * maha;
      rv = fast_exp2((float)(ll - lz2));
    }
    if (g == 0) {
      if constexpr (FIRST) nk += rv;
      rx[c] = rv;
    }
    asm volatile("s_waitcnt lgkmcnt(0)" ::: "memory");
    // sig_outer[d1][d2] += sum_rows (r x_d1) x_d2 on the bf16 matrix cores, 16 rows per
    // step: a = r x (fp32, as an fp32 step forms it) and x split exactly into three
    // bf16 values each, the six products of significance at least 2^-16 added smallest
    // first (error near an fp32 step's).  Lane (c, g) of step p holds rows
    // 16p + 8g + e of column c of each 32-coordinate block; steps whose 16 rows carry
    // no responsibility are skipped.
    const unsigned nz = (unsigned)__builtin_amdgcn_ballot_w64(rv != 0.0f);
#pragma unroll
    for (int p = 0; p < 2; ++p) {
      if (!dense && ((nz >> (16 * p)) & 0xffffu) == 0u) continue;
      const int rb = 16 * p + 8 * g;
      float rr[8];
#pragma unroll
      for (int e = 0; e < 8; ++e) rr[e] = rx[rb + e];
      bf16x8 bx[NMB][3], ba[NMB][3];
#pragma unroll
      for (int mb = 0; mb < NMB; ++mb) {
        float v[8], a[8];
#pragma unroll
        for (int e = 0; e < 8; ++e) {
          v[e] = xt[(rb + e) * RS + 32 * mb + c];
          a[e] = rr[e] * v[e];
        }
        if constexpr (FIRST) {
#pragma unroll
          for (int e = 0; e < 8; ++e) mua[mb] += a[e];
        }
        split3_bf16(f32x4{v[0], v[1], v[2], v[3]}, f32x4{v[4], v[5], v[6], v[7]}, bx[mb]);
        split3_bf16(f32x4{a[0], a[1], a[2], a[3]}, f32x4{a[4], a[5], a[6], a[7]}, ba[mb]);
      }
#pragma unroll
      for (int m1 = 0; m1 < NMB; ++m1) {
#pragma unroll
        for (int m2 = m1; m2 < NMB; ++m2) {
          const int sb = m1 * NMB - m1 * (m1 - 1) / 2 + (m2 - m1);   // upper-block index of (m1, m2)
          if (sb >= SB0 && sb < SB1) {
            f32x16& t = acc[sb - SB0];
            t = mfma_bf16(ba[m1][2], bx[m2][0], t);
            t = mfma_bf16(ba[m1][1], bx[m2][1], t);
            t = mfma_bf16(ba[m1][0], bx[m2][2], t);
            t = mfma_bf16(ba[m1][1], bx[m2][0], t);
            t = mfma_bf16(ba[m1][0], bx[m2][1], t);
            t = mfma_bf16(ba[m1][0], bx[m2][0], t);
          }
        }
      }
    }
    if (!PREFETCH) cnt_next = take(en);
    e = en;
    cnt = cnt_next;
  }

  const int64_t pbase = (int64_t)slab * KP + k;
  float* ps = part_sig + pbase * NSB * 1024;
#pragma unroll
  for (int sb = SB0; sb < SB1; ++sb) {
#pragma unroll
    for (int i = 0; i < 16; ++i) ps[sb * 1024 + acc_row(i, g) * 32 + c] = acc[sb - SB0][i];
  }
  if constexpr (FIRST) {
#pragma unroll
    for (int mb = 0; mb < NMB; ++mb) {
      const float v = mua[mb] + __shfl_xor(mua[mb], 32);
      if (g == 0) part_mu[pbase * DP + 32 * mb + c] = v;
    }
    float nks = nk;
#pragma unroll
    for (int o = 16; o >= 1; o >>= 1) nks += __shfl_xor(nks, o);
    if (lane == 0) part_nk[pbase] = nks;
  }
}

// ---------------------------------------------------------------------------
// Pass 2 of the stored branch (FGMM_FLAG_STORE_LOGJOINT_AUTO, D <= 64): r from the
// log-joint that pass 1 kept beside its need masks, over the default plan's slabs
// and partials.  One workgroup per (row slab, group of 8 components), one component
// per wave, so each 32-row X tile serves eight components: its fp32 rows, the eight
// components' log-joint columns and the rows' logZ2 reach LDS by buffer-to-LDS loads
// (four stages); every wave issues the same number of loads per tile (loads that
// only keep the count go out of range into a pad line), so the wait before each
// barrier is a fixed count.  The waves split the next tile's rows exactly into three
// bf16 parts (the B operands of sig_outer, read transposed) while computing the
// current one.  Per 16-row step, a = r x (fp32) is split as well and the six
// products of significance at least 2^-16 are added smallest first, as the
// gathering pass does; steps whose 16 rows carry no responsibility are skipped.
// `sel` is the probe's selector: the kernel returns unless it selects this branch.
// ---------------------------------------------------------------------------
constexpr int kFljWaves = 8;

template <int DP>
struct FljShape {
  static constexpr int NMB = DP / 32;
  static constexpr int XRS = DP + 4;                     // fp32 row stride of an X tile
  static constexpr int XPR = XRS / 4;                    // its 16-byte pieces per row (the last: padding)
  static constexpr int XPC = (32 * XPR + 63) / 64 * 64;  // pieces of the tile's region (whole waves)
  static constexpr int XQ = (XPC + 64 * kFljWaves - 1) / (64 * kFljWaves);
  static constexpr int PRS = DP + 16;                    // bf16 row stride of the split parts
  static constexpr int XB = XPC * 16;
  static constexpr int OFF_LJ = XB;                      // the 8 components' log-joint columns
  static constexpr int OFF_Z = XB + kFljWaves * 32 * 4;  // logZ2 of the 32 rows
  static constexpr int STAGE = OFF_Z + 32 * 8;
  static constexpr int NS = 4;
  static constexpr int PB = 3 * 32 * PRS * 2;            // one tile's split parts
  static constexpr int OFF_PARTS = NS * STAGE;
  static constexpr int OFF_R = OFF_PARTS + 2 * PB;       // r of the tile per wave
  static constexpr int OFF_PAD = OFF_R + kFljWaves * 32 * 4;
  static constexpr size_t lds = (size_t)OFF_PAD + 1024;
  // Loads of every wave per tile: XQ of X pieces, then 1 of log-joint columns (wave
  // 0), of logZ2 (wave 1) or into the pad line.
  static constexpr int NLOADS = XQ + 1;
};
__host__ inline int64_t flj_grid(int nslab, int ncg) { return (int64_t)8 * cdiv(nslab, 8) * ncg; }

template <int DP>
__global__ __attribute__((amdgpu_flat_work_group_size(64 * kFljWaves, 64 * kFljWaves), amdgpu_waves_per_eu(2, 2)))
void full_accum_ljt(const float* __restrict__ X, int64_t ldx, int64_t N, int D, int K, int KP,
                    const double* __restrict__ rowstat, const float* __restrict__ lj, int nslab,
                    int64_t rows_per_slab, int ncg, float* __restrict__ part_sig, float* __restrict__ part_mu,
                    float* __restrict__ part_nk, int dense, ProbeSel sel) {
  using SH = FljShape<DP>;
  constexpr int NMB = SH::NMB, NSB = NMB * (NMB + 1) / 2;
  constexpr int XRS = SH::XRS, PRS = SH::PRS, NS = SH::NS, NL = SH::NLOADS;
  static_assert(SH::lds <= 160 * 1024, "stages exceed LDS");
  if (!probe_selects(sel)) return;

  extern __shared__ __align__(16) unsigned char lds_raw[];
  const int tid = threadIdx.x, lane = tid & 63;
  const int wave = __builtin_amdgcn_readfirstlane(tid >> 6);
  const int c = lane & 31, g = lane >> 5;
  // Workgroup -> (slab, component group): the ncg groups of slab s run on XCD s % 8.
  const int xcd = blockIdx.x & 7, item = blockIdx.x >> 3;
  const int slab = (item / ncg) * 8 + xcd, cg = item % ncg;
  if (slab >= nslab) return;   // uniform over the workgroup
  const int k = cg * kFljWaves + wave;
  const bool active = k < K;

  const int64_t r_begin = (int64_t)slab * rows_per_slab;
  int64_t r_end = r_begin + rows_per_slab;
  if (r_end > N) r_end = N;
  const int ntiles = r_end > r_begin ? (int)cdiv(r_end - r_begin, 32) : 0;
  const int64_t tile0 = r_begin >> 5;   // rows_per_slab is a multiple of 32
  const int ncol = (D + 3) / 4;   // pieces of a row that hold columns below D
  // This lane's X pieces, offsets into the tile's rows (the host keeps 32 rows of
  // ldx under 2 GiB): slot q of wave w is LDS piece 64 (8 q + w) + lane of the tile
  // (row piece / XPR, column piece % XPR); the padding piece of each row, columns
  // past D and pieces past the tile read zeros.
  int xoff[SH::XQ];
#pragma unroll
  for (int q = 0; q < SH::XQ; ++q) {
    const int pc = (q * kFljWaves + wave) * 64 + lane;
    const int rr = pc / SH::XPR, cc = pc % SH::XPR;
    xoff[q] = (pc < 32 * SH::XPR && cc < ncol) ? (int)((int64_t)rr * ldx * 4 + cc * 16) : kBufOob;
  }
  unsigned char* const pad = lds_raw + SH::OFF_PAD;

  auto issue = [&](int t, auto stage_tag) __attribute__((always_inline)) {
    constexpr int S = decltype(stage_tag)::value;
    unsigned char* st = lds_raw + (size_t)S * SH::STAGE;
    const bool in = t < ntiles;
    const int64_t row0 = r_begin + (int64_t)t * 32;
    const int64_t nrow = in ? (r_end - row0 < 32 ? r_end - row0 : 32) : 0;
    const DmaSrc xsrc = dma_src(X + (in ? row0 : r_begin) * ldx, (uint32_t)(nrow * ldx * (int64_t)sizeof(float)));
#pragma unroll
    for (int q = 0; q < SH::XQ; ++q) {
      if ((q * kFljWaves + wave) * 64 < SH::XPC)
        lds_dma16(xsrc, st + (q * kFljWaves + wave) * 64 * 16, xoff[q], 0);
      else
        lds_dma16(xsrc, pad, kBufOob, 0);
    }
    const int64_t tg = tile0 + t;
    if (wave == 0) {
      // The group's 8 columns (out of range past KP).
      const int nk = KP - cg * kFljWaves < kFljWaves ? KP - cg * kFljWaves : kFljWaves;
      const DmaSrc lsrc = dma_src(lj + (in ? (tg * KP + cg * kFljWaves) * 32 : 0), in ? (uint32_t)(nk * 128) : 0u);
      if (lane < 8 * kFljWaves) lds_dma16(lsrc, st + SH::OFF_LJ, lane * 16, 0);   // 8 lanes per 128-byte column
    } else if (wave == 1) {
      const DmaSrc zsrc = dma_src(rowstat + (in ? row0 : 0), (uint32_t)(nrow * sizeof(double)));
      if (lane < 16) lds_dma16(zsrc, st + SH::OFF_Z, lane * 16, 0);
    } else {
      lds_dma16(xsrc, pad, kBufOob, 0);
    }
  };
  // The waves split tile t's fp32 rows (stage S) into parts buffer t & 1: lane
  // (wave, lane) takes pieces wave * 64 + lane + 512 j of the 32 x DP / 4.
  auto split = [&](int t, auto stage_tag) __attribute__((always_inline)) {
    constexpr int S = decltype(stage_tag)::value;
    const float* xs = reinterpret_cast<const float*>(lds_raw + (size_t)S * SH::STAGE);
    __bf16* pt = reinterpret_cast<__bf16*>(lds_raw + SH::OFF_PARTS + (t & 1) * SH::PB);
#pragma unroll
    for (int j = 0; j < (32 * DP / 4 + 64 * kFljWaves - 1) / (64 * kFljWaves); ++j) {
      const int pc = j * 64 * kFljWaves + tid;
      if (32 * DP / 4 % (64 * kFljWaves) == 0 || pc < 32 * DP / 4) {
        const int rr = pc / (DP / 4), cc = 4 * (pc % (DP / 4));
        const f32x4 v = *reinterpret_cast<const f32x4*>(xs + rr * XRS + cc);
        uint2 w[3];
#pragma unroll
        for (int h = 0; h < 2; ++h) {
          const f32x2 a = {v[2 * h], v[2 * h + 1]};
          const unsigned p1 = bf16_pair(a);
          const f32x2 d1 = a - bf16_pair_widen(p1);
          const unsigned p2 = bf16_pair(d1);
          const unsigned p3 = bf16_pair(d1 - bf16_pair_widen(p2));
          (h == 0 ? w[0].x : w[0].y) = p1;
          (h == 0 ? w[1].x : w[1].y) = p2;
          (h == 0 ? w[2].x : w[2].y) = p3;
        }
#pragma unroll
        for (int u = 0; u < 3; ++u) *reinterpret_cast<uint2*>(pt + (u * 32 + rr) * PRS + cc) = w[u];
      }
    }
  };

  f32x16 acc[NSB];
#pragma unroll
  for (int sb = 0; sb < NSB; ++sb) acc[sb] = zero16();
  float mua[NMB];
#pragma unroll
  for (int mb = 0; mb < NMB; ++mb) mua[mb] = 0.0f;
  float nk = 0.0f;
  float* rx = reinterpret_cast<float*>(lds_raw + SH::OFF_R) + wave * 32;

  auto compute = [&](int t, auto stage_tag) __attribute__((always_inline)) {
    constexpr int S = decltype(stage_tag)::value;
    const unsigned char* st = lds_raw + (size_t)S * SH::STAGE;
    const float* xt = reinterpret_cast<const float*>(st);
    const float l = reinterpret_cast<const float*>(st + SH::OFF_LJ)[wave * 32 + c];
    const double z = reinterpret_cast<const double*>(st + SH::OFF_Z)[c];
    const __bf16* pt = reinterpret_cast<const __bf16*>(lds_raw + SH::OFF_PARTS + (t & 1) * SH::PB);
    // r of row c (both half-waves hold it); 0 past the slab.
    const bool rin = r_begin + (int64_t)t * 32 + c < r_end;
    const float rv = (active && rin) ? fast_exp2((float)((double)l - z)) : 0.0f;
    if (g == 0) {
      nk += rv;
      rx[c] = rv;
    }
    const unsigned nz = (unsigned)__builtin_amdgcn_ballot_w64(rv != 0.0f);
    asm volatile("s_waitcnt lgkmcnt(0)" ::: "memory");
#pragma unroll
    for (int p = 0; p < 2; ++p) {
      if (!dense && ((nz >> (16 * p)) & 0xffffu) == 0u) continue;
      const int rb = 16 * p + 8 * g;
      const f32x4 r0 = *reinterpret_cast<const f32x4*>(rx + rb), r1 = *reinterpret_cast<const f32x4*>(rx + rb + 4);
      const float rr[8] = {r0[0], r0[1], r0[2], r0[3], r1[0], r1[1], r1[2], r1[3]};
      bf16x8 ba[NMB][3], bx[NMB][3];
#pragma unroll
      for (int mb = 0; mb < NMB; ++mb) {
        float a[8];
#pragma unroll
        for (int e = 0; e < 8; ++e) {
          a[e] = rr[e] * xt[(rb + e) * XRS + 32 * mb + c];
          mua[mb] += a[e];
        }
        split3_bf16(f32x4{a[0], a[1], a[2], a[3]}, f32x4{a[4], a[5], a[6], a[7]}, ba[mb]);
#pragma unroll
        for (int u = 0; u < 3; ++u) bx[mb][u] = lds_rows_operand(pt + u * 32 * PRS, PRS, 16 * p, 32 * mb, lane);
      }
#pragma unroll
      for (int m1 = 0; m1 < NMB; ++m1) {
#pragma unroll
        for (int m2 = m1; m2 < NMB; ++m2) {
          f32x16& a = acc[m1 * NMB - m1 * (m1 - 1) / 2 + (m2 - m1)];
          a = mfma_bf16(ba[m1][2], bx[m2][0], a);
          a = mfma_bf16(ba[m1][1], bx[m2][1], a);
          a = mfma_bf16(ba[m1][0], bx[m2][2], a);
          a = mfma_bf16(ba[m1][1], bx[m2][0], a);
          a = mfma_bf16(ba[m1][0], bx[m2][1], a);
          a = mfma_bf16(ba[m1][0], bx[m2][0], a);
        }
      }
    }
  };

  // Step t, stage S = t mod 4: issue tile t + 3, split tile t + 1 (its stage landed
  // at the last barrier), compute tile t (split during the previous step), wait for
  // tile t + 2's stage, barrier.
  auto step = [&](int t, auto stage_tag) __attribute__((always_inline)) {
    constexpr int S = decltype(stage_tag)::value;
    issue(t + 3, std::integral_constant<int, (S + 3) % NS>{});
    if (t + 1 < ntiles) split(t + 1, std::integral_constant<int, (S + 1) % NS>{});
    compute(t, stage_tag);
    vm_wait<NL>();
    __syncthreads();
  };
  if (ntiles > 0) {
    issue(0, std::integral_constant<int, 0>{});
    issue(1, std::integral_constant<int, 1>{});
    issue(2, std::integral_constant<int, 2>{});
    vm_wait<2 * NL>();   // tile 0
    __syncthreads();
    split(0, std::integral_constant<int, 0>{});
    vm_wait<NL>();       // tile 1
    __syncthreads();
  }
  using S0 = std::integral_constant<int, 0>;
  using S1 = std::integral_constant<int, 1>;
  using S2 = std::integral_constant<int, 2>;
  using S3 = std::integral_constant<int, 3>;
  for (int t = 0; t < ntiles; t += NS) {
    step(t, S0{});
    if (t + 1 >= ntiles) break;
    step(t + 1, S1{});
    if (t + 2 >= ntiles) break;
    step(t + 2, S2{});
    if (t + 3 >= ntiles) break;
    step(t + 3, S3{});
  }
  vm_wait<0>();   // no buffer-to-LDS load outlives the workgroup

  if (active) {
    const int64_t pbase = (int64_t)slab * KP + k;
    float* ps = part_sig + pbase * NSB * 1024;
#pragma unroll
    for (int sb = 0; sb < NSB; ++sb) {
#pragma unroll
      for (int i = 0; i < 16; ++i) ps[sb * 1024 + acc_row(i, g) * 32 + c] = acc[sb][i];
    }
#pragma unroll
    for (int mb = 0; mb < NMB; ++mb) {
      const float v = mua[mb] + __shfl_xor(mua[mb], 32);
      if (g == 0) part_mu[pbase * DP + 32 * mb + c] = v;
    }
    float nks = nk;
#pragma unroll
    for (int o = 16; o >= 1; o >>= 1) nks += __shfl_xor(nks, o);
    if (lane == 0) part_nk[pbase] = nks;
  }
}

template <int DP>
hipError_t launch_passes(const FullPlan& pl, const float* X, int64_t ldx, unsigned char* ws,
                         float* logZ, bool run1, bool run2, bool dense, hipStream_t stream) {
  const double* ck = reinterpret_cast<const double*>(ws + pl.off_ck);
  double* rowstat = reinterpret_cast<double*>(ws + pl.off_rowstat);
  float* lj = (pl.lj || pl.keep_lj || pl.autolj) ? reinterpret_cast<float*>(ws + pl.off_lj) : nullptr;
  auto set_lds = [](const void* f, size_t bytes) -> hipError_t {
    return bytes > 65536 ? hipFuncSetAttribute(f, hipFuncAttributeMaxDynamicSharedMemorySize, (int)bytes)
                         : hipSuccess;
  };
  // FGMM_FLAG_STORE_LOGJOINT_AUTO: the probe's counts select the branch in both passes.
  unsigned* probe = pl.autolj ? reinterpret_cast<unsigned*>(ws + pl.off_probe) : nullptr;
  const ProbeSel psel = probe ? ProbeSel{probe, pl.nprobe, probe_min_pairs(pl.N, pl.nprobe, (int)pl.K)}
                              : ProbeSel{nullptr, 0, 0};
  if (run1) {
    if constexpr (flj_applies(DP)) {
      if (pl.autolj) {
        // The probe's log-joints follow its counts in the workspace.
        float* lls = reinterpret_cast<float*>(ws + pl.off_probe + probe_bytes());
        hipLaunchKernelGGL((full_probe_ll<DP>), dim3((unsigned)(pl.nprobe * kProbeSplit)), dim3(64 * kProbeWaves), 0,
                           stream, X, ldx, pl.N, (int)pl.D, reinterpret_cast<const bf16x8*>(ws + pl.off_l3),
                           reinterpret_cast<const double*>(ws + pl.off_esw), ck, (int)pl.K, pl.KP, pl.nprobe, lls);
        hipLaunchKernelGGL(full_probe_count, dim3((unsigned)pl.nprobe), dim3(256), 0, stream, pl.N, (int)pl.K, pl.KP,
                           pl.nprobe, lls, probe);
      }
    }
    const size_t lds1 = full_x6_lds_bytes(DP) + (pl.needmode == kNeedLists ? full_list_lds_bytes(DP, pl.KP) : 0);
    // The stored plan runs up to D = 128 only; above, the default plan keeps the
    // log-joint beside the need masks (keep_lj) where it fits.
    // The need-mask instances, one per form.
    auto need_kern = [&](auto keep_tag) {
      constexpr bool KEEP = decltype(keep_tag)::value;
      return pl.needmode == kNeedLists    ? &full_lse_x6<DP, kLjmNeed, KEEP, kNeedLists>
             : pl.needmode == kNeedBounds ? &full_lse_x6<DP, kLjmNeed, KEEP, kNeedBounds>
                                          : &full_lse_x6<DP, kLjmNeed, KEEP, kNeedRunMax>;
    };
    auto kern = (DP > 128 || pl.need)
                    ? (DP > 128 && pl.keep_lj ? need_kern(std::integral_constant<bool, (DP > 128)>{})
                                              : need_kern(std::false_type{}))
                    : &full_lse_x6<DP, DP <= 128 ? kLjmStore : kLjmNeed>;
    hipError_t e = set_lds(reinterpret_cast<const void*>(kern), lds1);
    if (e != hipSuccess) return e;
    const unsigned grid1 = pl.need ? (unsigned)pl.grid1 : (unsigned)cdiv(pl.N, 32 * kWaves * full_x6_tpw(DP));
    hipLaunchKernelGGL(kern, dim3(grid1), dim3(kThreads), lds1, stream, X, ldx,
                       pl.N, (int)pl.D, reinterpret_cast<const bf16x8*>(ws + pl.off_l3),
                       reinterpret_cast<const double*>(ws + pl.off_esw), ck, (int)pl.K, pl.KP, logZ,
                       rowstat, lj, reinterpret_cast<unsigned*>(ws + pl.off_need),
                       reinterpret_cast<unsigned short*>(ws + pl.off_bound), dense ? 1 : 0, psel);
    if constexpr (flj_applies(DP)) {
      if (pl.autolj) {
        // The stored branch's instance: the same pass, keeping the log-joint and no need
        // masks (so no need-mask form).
        auto kst = &full_lse_x6<DP, kLjmNeed, true>;
        e = set_lds(reinterpret_cast<const void*>(kst), lds1);
        if (e != hipSuccess) return e;
        hipLaunchKernelGGL(kst, dim3(grid1), dim3(kThreads), lds1, stream, X, ldx, pl.N, (int)pl.D,
                           reinterpret_cast<const bf16x8*>(ws + pl.off_l3),
                           reinterpret_cast<const double*>(ws + pl.off_esw), ck, (int)pl.K, pl.KP, logZ, rowstat,
                           lj, reinterpret_cast<unsigned*>(ws + pl.off_need),
                           reinterpret_cast<unsigned short*>(ws + pl.off_bound), dense ? 1 : 0, psel);
      }
    }
  }
  if (!run2) return hipGetLastError();
  float* psig = reinterpret_cast<float*>(ws + pl.off_part_sig);
  float* pmu = reinterpret_cast<float*>(ws + pl.off_part_mu);
  float* pnk = reinterpret_cast<float*>(ws + pl.off_part_nk);
  const dim3 grid2((unsigned)(pl.nslab * pl.ncg));
  {
    if (pl.need) {
      constexpr size_t lds2 = gather_lds_bytes<DP>();
      static_assert(lds2 <= 160 * 1024, "gathering pass 2 exceeds LDS");
      auto launch = [&](auto grp_tag) -> hipError_t {
        constexpr int GRP = decltype(grp_tag)::value;
        if constexpr (GRP < gather_sig_groups(DP)) {
          auto kern2 = (DP > 128 && pl.keep_lj) ? &full_accum_gather<DP, GRP, (DP > 128)> : &full_accum_gather<DP, GRP>;
          hipError_t e = set_lds(reinterpret_cast<const void*>(kern2), lds2);
          if (e != hipSuccess) return e;
          hipLaunchKernelGGL(kern2, dim3((unsigned)gather_grid(pl.nslab, (int)pl.K)),
                             dim3(64 * kGatherWaves), lds2, stream, X, ldx, pl.N, (int)pl.D,
                             reinterpret_cast<const bf16x8*>(ws + pl.off_l3),
                             reinterpret_cast<const double*>(ws + pl.off_esw), ck, (int)pl.K, pl.KP, rowstat,
                             reinterpret_cast<const unsigned*>(ws + pl.off_need), pl.nslab, pl.rows_per_slab,
                             psig, pmu, pnk, dense ? 1 : 0, lj, psel);
        }
        return hipSuccess;
      };
      if constexpr (flj_applies(DP)) {
        if (pl.autolj) {
          using SH = FljShape<DP>;
          hipError_t ej = set_lds(reinterpret_cast<const void*>(&full_accum_ljt<DP>), SH::lds);
          if (ej != hipSuccess) return ej;
          const int ncg = (int)cdiv(pl.K, kFljWaves);
          hipLaunchKernelGGL((full_accum_ljt<DP>), dim3((unsigned)flj_grid(pl.nslab, ncg)), dim3(64 * kFljWaves),
                             SH::lds, stream, X, ldx, pl.N, (int)pl.D, (int)pl.K, pl.KP, rowstat, lj, pl.nslab,
                             pl.rows_per_slab, ncg, psig, pmu, pnk, dense ? 1 : 0, psel);
        }
      }
      hipError_t e = launch(std::integral_constant<int, 0>{});
      if (e == hipSuccess) e = launch(std::integral_constant<int, 1>{});
      if (e == hipSuccess) e = launch(std::integral_constant<int, 2>{});
      if (e == hipSuccess) e = launch(std::integral_constant<int, 3>{});
      if (e != hipSuccess) return e;
      return hipGetLastError();
    }
  }
  if constexpr (DP > 128) {
    return hipErrorInvalidValue;   // the stored plan runs up to D = 128 only
  } else {
    constexpr size_t lds2 = accum_lds_bytes<DP>();
    hipError_t e = set_lds(reinterpret_cast<const void*>(&full_accum<DP>), lds2);
    if (e != hipSuccess) return e;
    hipLaunchKernelGGL((full_accum<DP>), grid2, dim3(kAccThreads), lds2, stream, X, ldx, pl.N, (int)pl.D,
                       (int)pl.K, pl.KP, rowstat, pl.nslab, pl.rows_per_slab, psig, pmu, pnk, dense ? 1 : 0, lj);
    return hipGetLastError();
  }
}

// ===========================================================================
// Above D = 256 (any D up to kFullMaxD).  The prologue writes pass 1's operands in
// full_x6_prep's layout (l3, esw, ck) from one workgroup per (component,
// 32-coordinate block), without staging the o_qj of every coordinate in LDS.
// Pass 1 (full_lse_wide) forms the whitening in the same centred split-bf16 form
// and chain order as full_lse_x6, but the rows' split operands are re-read (L2)
// and re-split for every group of kWideCG coordinate blocks instead of being held
// in registers; it stores the log-joint.  Pass 2 (full_accum_wide) reads r from
// it and accumulates sig_outer strip by strip.
// ===========================================================================
__global__ __launch_bounds__(256) void full_x6_prep_wide(const float* __restrict__ mu, int64_t ldmu,
                                                         const float* __restrict__ L, int64_t K, int D, int DP,
                                                         const float* __restrict__ lpi, bf16x8* __restrict__ l3,
                                                         double* __restrict__ esw, double* __restrict__ ck) {
  __shared__ double se[32];   // e_j of this block's coordinates
  const int NQ = DP / 16, NMB = DP / 32;
  const int64_t k = blockIdx.x / NMB;
  const int mb = (int)(blockIdx.x % NMB);
  const int tid = threadIdx.x, lane = tid & 63, wave = tid >> 6;
  const int c = lane & 31, g = lane >> 5;
  const bool valid = k < K;
  const float* Lk = L + k * (int64_t)D * D;
  // o_qj = sum over d in chunk q of L_dj mu_d, an fp64 fma chain in d order.
  auto o_of = [&](int q, int j) -> double {
    double o = 0.0;
    if (valid && j < D)
      for (int d = 16 * q; d < 16 * q + 16 && d < D; ++d) o = fma((double)Lk[(int64_t)d * D + j], (double)mu[k * ldmu + d], o);
    return o;
  };
  // e_j = sum_q fp32(o_qj) - b_j with b_j = sum_q o_qj, both summed in q order.
  if (tid < 32) {
    double b = 0.0, osum = 0.0;
    for (int q = 0; q < NQ; ++q) {
      const double o = o_of(q, 32 * mb + tid);
      osum += (double)(float)o;
      b += o;
    }
    se[tid] = osum - b;
  }
  // Operands of chunks q = wave, wave + 4, ...: L^T split three ways, then the
  // offset slot -o_qj in k slots 0..2 against x6c_ones.
  const int j = 32 * mb + c;
  for (int q = wave; q < NQ; q += 4) {
    f32x4 lo = zero4(), hi = zero4();
#pragma unroll
    for (int e = 0; e < 4; ++e) {
      const int d0 = 16 * q + 8 * g + e, d1 = d0 + 4;
      lo[e] = (valid && d0 < D && j < D) ? Lk[(int64_t)d0 * D + j] : 0.0f;
      hi[e] = (valid && d1 < D && j < D) ? Lk[(int64_t)d1 * D + j] : 0.0f;
    }
    bf16x8 sp[3];
    split3_bf16(lo, hi, sp);
    bf16x8* dst = l3 + (((k * NMB + mb) * NQ + q) * 4) * 64 + lane;
#pragma unroll
    for (int t = 0; t < 3; ++t) dst[t * 64] = sp[t];
    const float mo = -(float)o_of(q, j);
    const f32x4 olo = {g == 0 ? mo : 0.0f, 0.0f, 0.0f, 0.0f};
    bf16x8 os[3];
    split3_bf16(olo, zero4(), os);
    bf16x8 ov;
#pragma unroll
    for (int e = 0; e < 8; ++e) ov[e] = (__bf16)0.0f;
    ov[0] = os[0][0];
    ov[1] = os[1][0];
    ov[2] = os[2][0];
    dst[3 * 64] = ov;
  }
  __syncthreads();
  if (tid < 32) {
    const int gg = tid >> 4, i = tid & 15;
    esw[(k * NMB + mb) * 32 + gg * 16 + i] = se[acc_row(i, gg)];
  }
  // c_k, the log-determinant summed in d order.
  if (mb == 0 && tid == 0) {
    double c0 = -INFINITY;
    if (valid) {
      double ld = 0.0;
      for (int d = 0; d < D; ++d) ld += log(fabs((double)Lk[(int64_t)d * D + d]) + 1e-30);
      c0 = ((double)lpi[k] + ld - 0.5 * (double)D * kLog2Pi) * kLog2e;
    }
    ck[k] = c0;
  }
}

// Pass-1 stage: the operands of kWideCG coordinate blocks x two chunks (4 splits
// each) of one component, and the blocks' e values and c_k.
__host__ __device__ constexpr int wide_stage_ops() { return kWideCG * 2 * 4 * 64; }   // bf16x8
__host__ __device__ constexpr int wide_stage_e() { return kWideCG * 32 + 8; }          // doubles
__host__ __device__ constexpr size_t wide_lse_lds_bytes() {
  return (size_t)2 * (wide_stage_ops() * sizeof(bf16x8) + wide_stage_e() * sizeof(double));
}

// One workgroup of kWideWaves1 waves per 32 kWideWaves1 rows; wave w owns tile
// blockIdx.x kWideWaves1 + w (lane = row, both half-waves).  Stage s = (k ngrp +
// grp) NQ/2 + qp runs chunks 2 qp and 2 qp + 1 of coordinate group grp of
// component k for every block of the group: seven bf16 steps per (block, chunk) in
// x6c_tile's order on the block's one accumulation chain, so each block's t equals
// what full_lse_x6 forms.  After a group's last chunk pair its blocks' (t + e)^2
// are added to maha in block order; after the component's last group the
// log-joint is stored and the online log-sum-exp advances.
__global__ __attribute__((amdgpu_flat_work_group_size(64 * kWideWaves1, 64 * kWideWaves1),
                          amdgpu_waves_per_eu(2, 2)))
void full_lse_wide(const float* __restrict__ X, int64_t ldx, int64_t N, int D, int DP,
                   const bf16x8* __restrict__ l3, const double* __restrict__ esw,
                   const double* __restrict__ ck, int K, int KP, float* __restrict__ logZ,
                   double* __restrict__ rowstat, float* __restrict__ lj) {
  constexpr int T = 64 * kWideWaves1;
  constexpr int SO = wide_stage_ops();
  constexpr int LPT = SO / T;               // one coordinate block per fetch register
  constexpr int NE = kWideCG * 32;
  constexpr int BW = wide_stage_e();
  static_assert(SO == LPT * T && T == 512 && LPT == kWideCG, "fetch index u is the block of the group");

  extern __shared__ __align__(16) unsigned char lds_raw[];
  bf16x8* l_l = reinterpret_cast<bf16x8*>(lds_raw);                              // [2][SO]
  double* e_l = reinterpret_cast<double*>(lds_raw + 2 * SO * sizeof(bf16x8));   // [2][BW]

  const int NMB = DP / 32, NQ = DP / 16, NQH = NQ / 2;
  const int ngrp = (NMB + kWideCG - 1) / kWideCG;
  const int tid = threadIdx.x, lane = tid & 63;
  const int wave = __builtin_amdgcn_readfirstlane(tid >> 6);
  const int c = lane & 31, g = lane >> 5;
  const int64_t tile = (int64_t)blockIdx.x * kWideWaves1 + wave;
  const int64_t row = tile * 32 + c;
  const bool valid = row < N;
  const int64_t nstage = (int64_t)K * ngrp * NQH;

  // Stage s -> component, group, chunk pair.
  auto decode = [&](int64_t s, int64_t& k, int& grp, int& qp) {
    qp = (int)(s % NQH);
    const int64_t kg = s / NQH;
    grp = (int)(kg % ngrp);
    k = kg / ngrp;
  };
  bf16x8 st[LPT];
  double est = 0.0;
  auto fetch = [&](int64_t s) {
    int64_t k;
    int grp, qp;
    decode(s, k, grp, qp);
    const int mb0 = grp * kWideCG;
    const int cnt = NMB - mb0 < kWideCG ? NMB - mb0 : kWideCG;
    // Register u holds block mb0 + u: (chunk 2 qp + (tid >> 8) & 1, split (tid >> 6) & 3, lane).
    const int qq = (tid >> 8) & 1, sp = (tid >> 6) & 3;
#pragma unroll
    for (int u = 0; u < LPT; ++u) {
      if (u < cnt) {
        st[u] = l3[(((k * NMB + mb0 + u) * NQ + 2 * qp + qq) * 4 + sp) * 64 + lane];
      } else {
#pragma unroll
        for (int e = 0; e < 8; ++e) st[u][e] = (__bf16)0.0f;
      }
    }
    if (tid < NE) est = tid < cnt * 32 ? esw[(k * NMB + mb0) * 32 + tid] : 0.0;
    else if (tid == NE) est = ck[k];
  };
  auto commit = [&](int buf) {
#pragma unroll
    for (int u = 0; u < LPT; ++u) l_l[buf * SO + u * T + tid] = st[u];
    if (tid <= NE) e_l[buf * BW + tid] = est;
  };
  // This lane's row, dimensions 16q + 8g .. +7 of the stage's two chunks.
  f32x4 raw[4];
  auto loadx = [&](int64_t s) {
    const int qp = (int)(s % NQH);
#pragma unroll
    for (int qq = 0; qq < 2; ++qq) {
      const int d0 = 16 * (2 * qp + qq) + 8 * g;
      raw[2 * qq] = load_row4(X, ldx, row, d0, D, valid);
      raw[2 * qq + 1] = load_row4(X, ldx, row, d0 + 4, D, valid);
    }
  };

  f32x16 acc[kWideCG];
#pragma unroll
  for (int u = 0; u < kWideCG; ++u) acc[u] = zero16();
  const bf16x8 ones = x6c_ones(lane);
  const double hl = 0.5 * kLog2e;
  double mx = -INFINITY, maha = 0.0;
  float sm = 0.0f;
  float* ljt = lj + tile * KP * 32 + c;

  if (nstage > 0) {
    fetch(0);
    loadx(0);
    commit(0);
  }
  __syncthreads();
  for (int64_t s = 0; s < nstage; ++s) {
    const int buf = (int)(s & 1);
    const bool more = s + 1 < nstage;
    int64_t k;
    int grp, qp;
    decode(s, k, grp, qp);
    const int cnt = NMB - grp * kWideCG < kWideCG ? NMB - grp * kWideCG : kWideCG;
    bf16x8 xb[2][3];
    split3_bf16(raw[0], raw[1], xb[0]);
    split3_bf16(raw[2], raw[3], xb[1]);
    if (more) {
      fetch(s + 1);
      loadx(s + 1);
    }
    const bf16x8* lc = l_l + buf * SO + lane;
#pragma unroll
    for (int u = 0; u < kWideCG; ++u) {
      if (u < cnt) {
#pragma unroll
        for (int qq = 0; qq < 2; ++qq) {
          bf16x8 a[4];
#pragma unroll
          for (int t = 0; t < 4; ++t) a[t] = lc[((u * 2 + qq) * 4 + t) * 64];
          // x6c_tile's steps: x2 mu2, x1 mu3, x3 mu1, x2 mu1, x1 mu2, -o, x1 mu1.
#pragma unroll
          for (int step = 0; step < 7; ++step) {
            const bf16x8 A = step == 0 ? a[1] : step == 1 ? a[2] : step <= 3 ? a[0]
                           : step == 4 ? a[1] : step == 5 ? a[3] : a[0];
            const bf16x8 B = step == 0 ? xb[qq][1] : step == 1 ? xb[qq][0] : step == 2 ? xb[qq][2]
                           : step == 3 ? xb[qq][1] : step == 4 ? xb[qq][0] : step == 5 ? ones : xb[qq][0];
            acc[u] = mfma_bf16(A, B, acc[u]);
          }
        }
      }
    }
    if (qp == NQH - 1) {   // the group's blocks are complete
      const double* ec = e_l + buf * BW;
#pragma unroll
      for (int u = 0; u < kWideCG; ++u) {
        if (u < cnt) {
          const double* eb = ec + u * 32 + g * 16;
#pragma unroll
          for (int i = 0; i < 16; ++i) {
            const double v = (double)acc[u][i] + eb[i];
            maha = fma(v, v, maha);
          }
        }
        acc[u] = zero16();
      }
      if (grp == ngrp - 1) {   // component k is complete
        maha += __shfl_xor(maha, 32);
        const double ll = ec[NE] - hl * maha;
        if (valid && g == 0) ljt[k * 32] = (float)ll;
        const double mn = fmax(mx, ll);
        const double ms = (mn == -INFINITY) ? 0.0 : mn;
        sm = sm * fast_exp2((float)(mx - ms)) + fast_exp2((float)(ll - ms));
        mx = mn;
        maha = 0.0;
      }
    }
    if (more) commit(buf ^ 1);
    lds_barrier();
  }
  const double lz2 = mx + (double)log2f(sm);
  if (valid && g == 0) {
    rowstat[row] = lz2;
    if (logZ) logZ[row] = (float)(lz2 * kLn2);
  }
}

// Pass 2 above D = 256: one wave per (row slab, component, strip), where strip
// (b1, b2s) holds the upper blocks (b1, b2), b2s <= b2 < b2s + kWideSW, of one
// block row of sig_outer; the strips of a (slab, component) are dealt in fours to
// workgroups.  Per 32-row tile the lanes form r = 2^(ll2 - logZ2) from the stored
// log-joint; tiles and 16-row steps with no nonzero r are skipped.  Each step forms
// a = r x over block b1 and accumulates a x^T into every block of the strip as six
// split-bf16 products (the gathering pass 2's order); the strip starting on the
// diagonal also sums mu_acc of block b1, and strip 0 Nk.  Rows are read from L2
// (each 32-column slice of a row is one 128-byte line per 32 lanes).
__global__ __launch_bounds__(64 * kWideWaves2)
void full_accum_wide(const float* __restrict__ X, int64_t ldx, int64_t N, int D, int DP, int K, int KP,
                     const double* __restrict__ rowstat, const float* __restrict__ lj, int nslab,
                     int64_t rows_per_slab, int nstrip, float* __restrict__ part_sig,
                     float* __restrict__ part_mu, float* __restrict__ part_nk, int dense) {
  __shared__ float r_all[kWideWaves2][32];
  const int NMB = DP / 32;
  const int64_t NSB = (int64_t)NMB * (NMB + 1) / 2;
  const int tid = threadIdx.x, lane = tid & 63;
  const int wave = __builtin_amdgcn_readfirstlane(tid >> 6);
  const int c = lane & 31, g = lane >> 5;
  const int nsg = (nstrip + kWideWaves2 - 1) / kWideWaves2;
  const int sgp = (int)(blockIdx.x % nsg);
  const int64_t rest = blockIdx.x / nsg;
  const int k = (int)(rest % K);
  const int slab = (int)(rest / K);
  const int strip = sgp * kWideWaves2 + wave;
  if (strip >= nstrip || slab >= nslab) return;   // no barrier in this kernel
  int b1 = 0, sr = strip;
  for (;;) {
    const int ns = (NMB - b1 + kWideSW - 1) / kWideSW;
    if (sr < ns) break;
    sr -= ns;
    ++b1;
  }
  const int b2s = b1 + sr * kWideSW;
  const int cnt = NMB - b2s < kWideSW ? NMB - b2s : kWideSW;
  const bool first = b2s == b1;   // forms mu_acc of block b1
  const bool nkw = strip == 0;    // forms Nk

  const int64_t r_begin = (int64_t)slab * rows_per_slab;
  int64_t r_end = r_begin + rows_per_slab;
  if (r_end > N) r_end = N;

  f32x16 acc[kWideSW];
#pragma unroll
  for (int j = 0; j < kWideSW; ++j) acc[j] = zero16();
  float mua = 0.0f, nk = 0.0f;
  float* rx = r_all[wave];
  const int cb1 = 32 * b1 + c;
  auto xval = [&](int64_t rw, int col) -> float {
    return (rw < r_end && col < D) ? X[rw * ldx + col] : 0.0f;
  };

  for (int64_t r0 = r_begin; r0 < r_end; r0 += 32) {
    const int64_t row = r0 + c;
    float rv = 0.0f;
    if (row < r_end) {
      const float l = lj[((row >> 5) * KP + k) * 32 + (row & 31)];
      rv = fast_exp2((float)((double)l - rowstat[row]));
    }
    if (nkw && g == 0) nk += rv;
    const unsigned nz = (unsigned)__builtin_amdgcn_ballot_w64(rv != 0.0f);   // lanes 0..31: rows
    if (!dense && nz == 0u) continue;
    if (g == 0) rx[c] = rv;
    __builtin_amdgcn_wave_barrier();
#pragma unroll
    for (int p = 0; p < 2; ++p) {
      if (!dense && ((nz >> (16 * p)) & 0xffffu) == 0u) continue;
      const int rb = 16 * p + 8 * g;   // this lane's rows rb .. rb + 7 of the tile
      float a[8];
#pragma unroll
      for (int e = 0; e < 8; ++e) {
        a[e] = rx[rb + e] * xval(r0 + rb + e, cb1);
        if (first) mua += a[e];
      }
      bf16x8 ba[3];
      split3_bf16(f32x4{a[0], a[1], a[2], a[3]}, f32x4{a[4], a[5], a[6], a[7]}, ba);
#pragma unroll
      for (int j = 0; j < kWideSW; ++j) {
        if (j < cnt) {
          const int col = 32 * (b2s + j) + c;
          float v[8];
#pragma unroll
          for (int e = 0; e < 8; ++e) v[e] = xval(r0 + rb + e, col);
          bf16x8 bx[3];
          split3_bf16(f32x4{v[0], v[1], v[2], v[3]}, f32x4{v[4], v[5], v[6], v[7]}, bx);
          f32x16& t = acc[j];
          t = mfma_bf16(ba[2], bx[0], t);
          t = mfma_bf16(ba[1], bx[1], t);
          t = mfma_bf16(ba[0], bx[2], t);
          t = mfma_bf16(ba[1], bx[0], t);
          t = mfma_bf16(ba[0], bx[1], t);
          t = mfma_bf16(ba[0], bx[0], t);
        }
      }
    }
    __builtin_amdgcn_wave_barrier();
  }

  const int64_t pbase = (int64_t)slab * KP + k;
  float* ps = part_sig + pbase * NSB * 1024;
  const int64_t sb0 = (int64_t)b1 * NMB - (int64_t)b1 * (b1 - 1) / 2 + (b2s - b1);
#pragma unroll
  for (int j = 0; j < kWideSW; ++j) {
    if (j < cnt) {
#pragma unroll
      for (int i = 0; i < 16; ++i) ps[(sb0 + j) * 1024 + acc_row(i, g) * 32 + c] = acc[j][i];
    }
  }
  if (first) {
    const float v = mua + __shfl_xor(mua, 32);
    if (g == 0) part_mu[pbase * DP + cb1] = v;
  }
  if (nkw) {
    float nks = nk;
#pragma unroll
    for (int o = 16; o >= 1; o >>= 1) nks += __shfl_xor(nks, o);
    if (lane == 0) part_nk[pbase] = nks;
  }
}

hipError_t launch_wide(const FullPlan& pl, const float* X, int64_t ldx, unsigned char* ws, float* logZ,
                       bool run1, bool run2, bool dense, hipStream_t stream) {
  const double* ck = reinterpret_cast<const double*>(ws + pl.off_ck);
  double* rowstat = reinterpret_cast<double*>(ws + pl.off_rowstat);
  float* lj = reinterpret_cast<float*>(ws + pl.off_lj);
  if (run1) {
    constexpr size_t lds1 = wide_lse_lds_bytes();
    static_assert(lds1 <= (size_t)160 * 1024, "pass-1 stages fit LDS");
    hipError_t e = hipFuncSetAttribute(reinterpret_cast<const void*>(&full_lse_wide),
                                       hipFuncAttributeMaxDynamicSharedMemorySize, (int)lds1);
    if (e != hipSuccess) return e;
    hipLaunchKernelGGL(full_lse_wide, dim3((unsigned)cdiv(pl.N, 32 * kWideWaves1)), dim3(64 * kWideWaves1), lds1,
                       stream, X, ldx, pl.N, (int)pl.D, pl.DP, reinterpret_cast<const bf16x8*>(ws + pl.off_l3),
                       reinterpret_cast<const double*>(ws + pl.off_esw), ck, (int)pl.K, pl.KP, logZ, rowstat, lj);
  }
  if (!run2) return hipGetLastError();
  const int64_t nsg = cdiv(pl.nstrip, kWideWaves2);
  hipLaunchKernelGGL(full_accum_wide, dim3((unsigned)((int64_t)pl.nslab * pl.K * nsg)), dim3(64 * kWideWaves2), 0,
                     stream, X, ldx, pl.N, (int)pl.D, pl.DP, (int)pl.K, pl.KP, rowstat, lj, pl.nslab,
                     pl.rows_per_slab, pl.nstrip, reinterpret_cast<float*>(ws + pl.off_part_sig),
                     reinterpret_cast<float*>(ws + pl.off_part_mu), reinterpret_cast<float*>(ws + pl.off_part_nk),
                     dense ? 1 : 0);
  return hipGetLastError();
}

// ===========================================================================
// bf16 operand contract (FGMM_FLAG_BF16), the arithmetic of the reference's full
// H100 kernels (flash_gmm_full_h100.py:71-139 pass 1, :146-228 pass 2, :289-298
// constants), in log2 units:
//   b_k = L_k^T mu_k (fp32),  c_k = (lpi_k + sum_d log(|L_k,dd| + 1e-30) - 0.5 D log 2pi) log2 e
//   v = bf16(x) . bf16(L_k) - b_k,  maha = ||v||^2,  ll2 = c_k - 0.5 log2 e maha   (fp32)
//   r = 2^(ll2 - logZ2);  Nk = sum r;  mu_acc = bf16(r)^T bf16(x)
//   sig_outer_k[d2][d1] = sum_n bf16(r_nk x_n,d2) bf16(x_n,d1)   (not symmetric)
// Pass 1 whitens on v_mfma_f32_32x32x16_bf16 (V^T = bf16(L)^T bf16(X)^T: lane = row,
// 16 whitened coordinates per register block) and stores the fp32 log-joint; pass 2
// reads it back.  Pass 2 forms the A operand bf16(r x_d2) in registers from fp32 X
// tiles and accumulates every 32x32 block of sig_outer; mu_acc is one more matrix
// step per row step whose A operand holds bf16(r) of the workgroup's components.
// ===========================================================================

// Prologue, one 64-thread block per component (k < KP):
//   lop[k][mb][q][lane] (bf16x8) = bf16(L[k][16q + 8g + e][32 mb + c]), the A operand
//   bsw[k][mb][g][i]    (fp32)   = b[k][32 mb + acc_row(i, g)]
//   ck[k]               (fp32)
__global__ __launch_bounds__(64) void full_bf16_prep(const float* __restrict__ mu, int64_t ldmu,
                                                     const float* __restrict__ L, int64_t K, int D,
                                                     int DP, const float* __restrict__ lpi,
                                                     bf16x8* __restrict__ lop, float* __restrict__ bsw,
                                                     float* __restrict__ ck) {
  __shared__ double sb[128];   // DP <= 128
  const int64_t k = blockIdx.x;
  const int lane = threadIdx.x, c = lane & 31, g = lane >> 5;
  const bool valid = k < K;
  const float* Lk = L + k * (int64_t)D * D;
  for (int j = lane; j < DP; j += 64) {
    double b = 0.0;
    if (valid && j < D)
#pragma unroll 8
      for (int i = 0; i < D; ++i) b = fma((double)Lk[(int64_t)i * D + j], (double)mu[k * ldmu + i], b);
    sb[j] = b;
  }
  if (lane == 0) {
    double c0 = -INFINITY;
    if (valid) {
      double ld = 0.0;
#pragma unroll 8
      for (int d = 0; d < D; ++d) ld += log(fabs((double)Lk[(int64_t)d * D + d]) + 1e-30);
      c0 = ((double)lpi[k] + ld - 0.5 * (double)D * kLog2Pi) * kLog2e;
    }
    ck[k] = (float)c0;
  }
  const int NMB = DP / 32, NQ = DP / 16;
  for (int mb = 0; mb < NMB; ++mb) {
    const int j = 32 * mb + c;
    for (int q = 0; q < NQ; ++q) {
      bf16x8 v;
#pragma unroll
      for (int e = 0; e < 8; ++e) {
        const int i = 16 * q + 8 * g + e;
        v[e] = (__bf16)((valid && i < D && j < D) ? Lk[(int64_t)i * D + j] : 0.0f);
      }
      lop[((k * NMB + mb) * NQ + q) * 64 + lane] = v;
    }
  }
  __syncthreads();
  for (int mb = 0; mb < NMB; ++mb) {
    if (lane < 32) {
      const int gg = lane >> 4, i = lane & 15;
      bsw[(k * NMB + mb) * 32 + gg * 16 + i] = (float)sb[32 * mb + acc_row(i, gg)];
    }
  }
}

// Pass 1: grid over 128-row tiles, 4 waves of 32 rows; one component's bf16 L^T, b
// and c stream through an LDS double buffer.  Writes logZ, logZ2 and the log-joint.
template <int DP>
constexpr size_t bf16_lse_lds_bytes() {
  return (size_t)2 * DP * DP * 2 + (size_t)2 * (DP + 4) * sizeof(float);
}

template <int DP>
__global__ __launch_bounds__(kThreads) void full_bf16_lse(const float* __restrict__ X, int64_t ldx,
                                                          int64_t N, int D,
                                                          const bf16x8* __restrict__ lop,
                                                          const float* __restrict__ bsw,
                                                          const float* __restrict__ ck, int K, int KP,
                                                          float* __restrict__ logZ,
                                                          float* __restrict__ rowstat,
                                                          float* __restrict__ lj) {
  constexpr int NMB = DP / 32, NQ = DP / 16;
  constexpr int BLK = NMB * NQ * 64;              // bf16x8 per component
  constexpr int LPT = (BLK + kThreads - 1) / kThreads;
  constexpr int BW = DP + 4;                      // floats per component stage (b, then c)

  extern __shared__ __align__(16) unsigned char lds_raw[];
  bf16x8* l_l = reinterpret_cast<bf16x8*>(lds_raw);                                // [2][BLK]
  float* b_l = reinterpret_cast<float*>(lds_raw + 2 * BLK * sizeof(bf16x8));       // [2][BW]

  const int tid = threadIdx.x, lane = tid & 63, wave = tid >> 6;
  const int c = lane & 31, g = lane >> 5;
  const int64_t tile = (int64_t)blockIdx.x * kWaves + wave;   // 32-row tile
  const int64_t row = tile * 32 + c;
  const bool valid = row < N;
  float* ljt = lj + tile * KP * 32 + c;

  bf16x8 st[LPT];
  float bst = 0.0f;
  auto fetch = [&](int k) {
    const bf16x8* src = lop + (int64_t)k * BLK;
#pragma unroll
    for (int q = 0; q < LPT; ++q)
      if (BLK % kThreads == 0 || q * kThreads + tid < BLK) st[q] = src[q * kThreads + tid];
    if (tid < DP) bst = bsw[(int64_t)k * DP + tid];
    else if (tid == DP) bst = ck[k];
  };
  auto commit = [&](int buf) {
#pragma unroll
    for (int q = 0; q < LPT; ++q)
      if (BLK % kThreads == 0 || q * kThreads + tid < BLK) l_l[buf * BLK + q * kThreads + tid] = st[q];
    if (tid <= DP) b_l[buf * BW + tid] = bst;
  };
  fetch(0);
  // B operand: this lane's row, dimensions 16q + 8g + e, rounded to bf16.
  bf16x8 xb[NQ];
#pragma unroll
  for (int q = 0; q < NQ; ++q) {
    const int d0 = 16 * q + 8 * g;
    xb[q] = to_bf16x8(load_row4(X, ldx, row, d0, D, valid), load_row4(X, ldx, row, d0 + 4, D, valid));
  }
  commit(0);
  lds_barrier();

  const float hl = (float)(0.5 * kLog2e);
  float mx = -INFINITY, sm = 0.0f;
  for (int k = 0; k < K; ++k) {
    const int buf = k & 1;
    const bool more = k + 1 < K;
    if (more) fetch(k + 1);
    const bf16x8* la = l_l + buf * BLK + lane;
    const float* bb = b_l + buf * BW + g * 16;
    float maha = 0.0f;
#pragma unroll
    for (int mb = 0; mb < NMB; ++mb) {
      // V^T block mb: lane = row, register i = coordinate 32 mb + acc_row(i, g).
      f32x16 v = zero16();
#pragma unroll
      for (int q = 0; q < NQ; ++q) v = mfma_bf16(la[(mb * NQ + q) * 64], xb[q], v);
#pragma unroll
      for (int i = 0; i < 16; ++i) {
        const float t = v[i] - bb[mb * 32 + i];
        maha = fmaf(t, t, maha);
      }
    }
    maha += __shfl_xor(maha, 32);
    const float ll = b_l[buf * BW + DP] - hl * maha;
    if (g == 0) ljt[k * 32] = ll;
    const float mn = fmaxf(mx, ll);
    const float ms = (mn == -INFINITY) ? 0.0f : mn;
    sm = sm * fast_exp2(mx - ms) + fast_exp2(ll - ms);
    mx = mn;
    if (more) commit(buf ^ 1);
    lds_barrier();
  }
  const float lz2 = mx + log2f(sm);
  if (valid && g == 0) {
    rowstat[row] = lz2;
    if (logZ) logZ[row] = lz2 * (float)kLn2;
  }
}

// Pass 2 layout: waves per component = NMB (wave owns the 32 rows d2 of block mb2 of
// sig_outer and all NMB column blocks), components per workgroup and row groups so
// that the 8 waves are used (D = 96: 6 of them).
__host__ __device__ constexpr int bf16_comps_per_wg(int NMB) { return NMB <= 2 ? 4 : 2; }
// Components per wave: each wave accumulates its column block for this many
// components from one staged X tile (their sig blocks take 64 or 128 registers).
__host__ __device__ constexpr int bf16_comp_reps(int NMB) { return NMB <= 2 ? 4 : 2; }
__host__ __device__ constexpr int bf16_row_groups(int NMB) { return NMB == 1 ? 2 : 1; }

// Row strides of pass 2's X tiles: fp32 DP + 4 words (rows r and r + 8 of one column,
// which one A-operand read takes for the two half-waves, fall 32 banks apart), bf16
// DP + 16 (an odd multiple of 32 bytes, for the transposing B-operand reads).
__host__ __device__ constexpr int bf16_xf_stride(int DP) { return DP + 4; }
__host__ __device__ constexpr int bf16_xh_stride(int DP) { return DP + 16; }

template <int DP>
constexpr size_t bf16_accum_lds_bytes() {
  constexpr int NMB = DP / 32;
  constexpr int TR = 32 * bf16_row_groups(NMB);
  return (size_t)2 * TR * bf16_xf_stride(DP) * sizeof(float)   // X tiles, fp32, row-major
         + (size_t)2 * TR * bf16_xh_stride(DP) * 2             // X tiles, bf16, row-major
         + (size_t)2 * TR * sizeof(float)                      // logZ2
         + (size_t)bf16_row_groups(NMB) * bf16_comps_per_wg(NMB) * bf16_comp_reps(NMB) * 32 * sizeof(float);   // r
}

// The X tiles are loaded coalesced and held row-major in LDS, in fp32 (for r x, which
// the contract forms in fp32 before rounding) and in bf16 (the B operands, two
// transposing reads each, lds_rows_operand).
template <int DP>
__global__ __attribute__((amdgpu_flat_work_group_size(kAccThreads, kAccThreads), amdgpu_waves_per_eu(2, 2)))
void full_bf16_accum(const float* __restrict__ X, int64_t ldx, int64_t N, int D, int K, int KP,
                     const float* __restrict__ rowstat, const float* __restrict__ lj, int nslab,
                     int64_t rows_per_slab, float* __restrict__ part_sig, float* __restrict__ part_mu,
                     float* __restrict__ part_nk, int dense) {
  constexpr int NMB = DP / 32;
  constexpr int CPWG = bf16_comps_per_wg(NMB);
  constexpr int RG = bf16_row_groups(NMB);
  constexpr int TR = 32 * RG;
  constexpr int V4 = DP / 4;
  constexpr int NV = TR * V4;                     // float4 per tile
  constexpr int LPT = (NV + kAccThreads - 1) / kAccThreads;
  static_assert(CPWG * NMB * RG <= kAccWaves, "waves cover the work");

  constexpr int XF = bf16_xf_stride(DP), XH = bf16_xh_stride(DP);
  extern __shared__ __align__(16) unsigned char lds_raw[];
  float* xf = reinterpret_cast<float*>(lds_raw);                           // [2][TR][XF]
  __bf16* xh = reinterpret_cast<__bf16*>(xf + 2 * TR * XF);                // [2][TR][XH]
  float* rs = reinterpret_cast<float*>(xh + 2 * TR * XH);                  // [2][TR]
  float* r_l = rs + 2 * TR;                                                // [8][32]

  const int tid = threadIdx.x, lane = tid & 63, wave = tid >> 6;
  const int c = lane & 31, g = lane >> 5;
  // wave = (rg * NMB + mb2) * CPWG + cw; wave cw serves the Q components cw Q + qi of the
  // workgroup's CQ = CPWG Q.
  constexpr int Q = bf16_comp_reps(NMB), CQ = CPWG * Q;
  static_assert(CQ <= 32, "components of the mu_acc step");
  const bool in_use = wave < CPWG * NMB * RG;     // D = 96 leaves two waves idle
  const int cw = wave % CPWG, mb2 = (wave / CPWG) % NMB, rg = in_use ? wave / (CPWG * NMB) : 0;
  const int slab = blockIdx.x % nslab;
  const int cg = blockIdx.x / nslab;
  const int k0 = cg * CQ + cw * Q;                // this wave's first component
  const bool active = in_use && k0 < K;
  const bool mu_wave = in_use && cw == 0;         // also accumulates mu_acc block mb2

  const int64_t r_begin = (int64_t)slab * rows_per_slab;
  int64_t r_end = r_begin + rows_per_slab;
  if (r_end > N) r_end = N;
  const int ntiles = r_end > r_begin ? (int)cdiv(r_end - r_begin, TR) : 0;

  f32x16 acc[Q][NMB];
#pragma unroll
  for (int qi = 0; qi < Q; ++qi) {
#pragma unroll
    for (int mb = 0; mb < NMB; ++mb) acc[qi][mb] = zero16();
  }
  f32x16 macc = zero16();
  float nk[Q];
#pragma unroll
  for (int qi = 0; qi < Q; ++qi) nk[qi] = 0.0f;

  f32x4 stage[LPT];
  float rstage = INFINITY;
  const bool full_d = (D == DP);
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
      rstage = (row < r_end) ? rowstat[row] : INFINITY;   // r = 0 past the slab
    }
  };
  auto commit = [&](int buf) {
    float* df = xf + buf * TR * XF;
    __bf16* dh = xh + buf * TR * XH;
    typedef __bf16 bf16x4 __attribute__((ext_vector_type(4)));
#pragma unroll
    for (int q = 0; q < LPT; ++q) {
      const int idx = q * kAccThreads + tid;
      if (NV % kAccThreads != 0 && idx >= NV) continue;
      const int r = tile_row(idx), d = tile_col(idx);
      const f32x4 v = stage[q];
      *reinterpret_cast<f32x4*>(df + r * XF + d) = v;
      *reinterpret_cast<bf16x4*>(dh + r * XH + d) = bf16x4{(__bf16)v.x, (__bf16)v.y, (__bf16)v.z, (__bf16)v.w};
    }
    if (tid < TR) rs[buf * TR + tid] = rstage;
  };

  // The stored log-joint of component k0 + qi for row c of tile t (0 past the slab or
  // past K, where logZ2 = +inf or the skipped store leave r = 0); loaded one tile ahead.
  // The mb2 = 0 wave of each component set forms r for the workgroup.
  const bool r_maker = active && mb2 == 0;
  auto lj_of = [&](int t, int qi) -> float {
    const int64_t row0 = r_begin + (int64_t)t * TR + rg * 32;
    return (r_maker && k0 + qi < K && row0 < r_end) ? lj[((row0 >> 5) * KP + k0 + qi) * 32 + c] : 0.0f;
  };
  float lnext[Q];
#pragma unroll
  for (int qi = 0; qi < Q; ++qi) lnext[qi] = 0.0f;
  if (ntiles > 0) {
    fetch(0);
#pragma unroll
    for (int qi = 0; qi < Q; ++qi) lnext[qi] = lj_of(0, qi);
    commit(0);
  }
  lds_barrier();

  float* r_rg = r_l + rg * CQ * 32;   // [row group][CQ][32]
  for (int t = 0; t < ntiles; ++t) {
    const int buf = t & 1;
    const bool more = t + 1 < ntiles;
    if (r_maker) {
#pragma unroll
      for (int qi = 0; qi < Q; ++qi) {
        const float rv = (k0 + qi < K) ? fast_exp2(lnext[qi] - rs[buf * TR + rg * 32 + c]) : 0.0f;
        if (g == 0) {
          r_rg[(cw * Q + qi) * 32 + c] = rv;
          nk[qi] += rv;
        }
      }
    }
    if (more) {
#pragma unroll
      for (int qi = 0; qi < Q; ++qi) lnext[qi] = lj_of(t + 1, qi);
      fetch(t + 1);
    }
    lds_barrier();
    const float* xa = xf + buf * TR * XF;
    const __bf16* xb = xh + buf * TR * XH;
#pragma unroll
    for (int p = 0; p < 2; ++p) {
      // Rows rg*32 + 16p + 8g + e of this step.
      const int r0 = rg * 32 + 16 * p;
      bf16x8 bop[NMB];
#pragma unroll
      for (int mb = 0; mb < NMB; ++mb) bop[mb] = in_use ? lds_rows_operand(xb, XH, r0, 32 * mb, lane) : bf16x8{};
      if (active) {
        // A = bf16(r x_d2): lane = d2 = 32 mb2 + c, elements = the 8 rows.
        const float* xx = xa + (r0 + 8 * g) * XF + 32 * mb2 + c;
        const f32x4 x0 = {xx[0], xx[XF], xx[2 * XF], xx[3 * XF]};
        const f32x4 x1 = {xx[4 * XF], xx[5 * XF], xx[6 * XF], xx[7 * XF]};
#pragma unroll
        for (int qi = 0; qi < Q; ++qi) {
          const f32x4* rr = reinterpret_cast<const f32x4*>(r_rg + (cw * Q + qi) * 32 + 16 * p + 8 * g);
          const bf16x8 a = to_bf16x8(rr[0] * x0, rr[1] * x1);
          // A step whose 16 rows x 32 coordinates of bf16(r x) are all zero adds nothing.
          if (dense || any_nonzero(a)) {
#pragma unroll
            for (int mb = 0; mb < NMB; ++mb) acc[qi][mb] = mfma_bf16(a, bop[mb], acc[qi][mb]);
          }
        }
      }
      if (mu_wave) {
        // A = bf16(r) of the workgroup's components (rows m = component), B = block mb2.
        bf16x8 a = {};
        if (c < CQ && cg * CQ + c < K) {
          const f32x4* rr = reinterpret_cast<const f32x4*>(r_rg + c * 32 + 16 * p + 8 * g);
          a = to_bf16x8(rr[0], rr[1]);
        }
        // B = column block mb2 (mb2 is not a compile-time index: read it again).
        const bf16x8 bm = lds_rows_operand(xb, XH, r0, 32 * mb2, lane);
        if (dense || any_nonzero(a)) macc = mfma_bf16(a, bm, macc);
      }
    }
    if (more) commit(buf ^ 1);
    lds_barrier();
  }

  const int64_t pbase0 = ((int64_t)slab * RG + rg) * KP + (int64_t)cg * CQ;
  if (active) {
#pragma unroll
    for (int qi = 0; qi < Q; ++qi) {
      if (k0 + qi >= K) continue;
      float* ps = part_sig + ((pbase0 + cw * Q + qi) * NMB * NMB + mb2 * NMB) * 1024;
#pragma unroll
      for (int mb = 0; mb < NMB; ++mb) {
#pragma unroll
        for (int i = 0; i < 16; ++i) ps[mb * 1024 + acc_row(i, g) * 32 + c] = acc[qi][mb][i];
      }
      if (mb2 == 0) {
        float s = nk[qi];
#pragma unroll
        for (int o = 16; o >= 1; o >>= 1) s += __shfl_xor(s, o);
        if (lane == 0) part_nk[pbase0 + cw * Q + qi] = s;
      }
    }
  }
  if (mu_wave) {
    // Register i of lane-half g holds component acc_row(i, g) of the workgroup.
#pragma unroll
    for (int i = 0; i < 16; ++i) {
      const int ci = acc_row(i, g);
      if (ci < CQ && cg * CQ + ci < K) part_mu[(pbase0 + ci) * DP + 32 * mb2 + c] = macc[i];
    }
  }
}

// Finish of the bf16 contract: every element of sig_outer from its own block (no
// mirroring), fixed-order fp64 sums over the partials.
__global__ __launch_bounds__(256) void full_bf16_reduce(const float* __restrict__ part_sig,
                                                        const float* __restrict__ part_mu,
                                                        const float* __restrict__ part_nk, int npart,
                                                        int KP, int DP, int NMB, int64_t K, int D,
                                                        float* __restrict__ Nk, float* __restrict__ mu_acc,
                                                        float* __restrict__ sig_outer, int accumulate) {
  const int NB2 = NMB * NMB;
  const int64_t idx = (int64_t)blockIdx.x * blockDim.x + threadIdx.x;
  const int64_t nsig = K * D * D;
  if (idx < nsig) {
    const int64_t k = idx / ((int64_t)D * D);
    const int rem = (int)(idx % ((int64_t)D * D));
    const int d2 = rem / D, d1 = rem % D;
    const int blk = (d2 / 32) * NMB + d1 / 32;
    const double s = strided_sum(part_sig + ((int64_t)k * NB2 + blk) * 1024 + (d2 % 32) * 32 + d1 % 32,
                                 npart, (int64_t)KP * NB2 * 1024);
    float* o = sig_outer + idx;
    *o = accumulate ? (float)((double)*o + s) : (float)s;
    return;
  }
  const int64_t j = idx - nsig;
  if (j < K * D) {
    const int64_t k = j / D;
    const int d = (int)(j % D);
    const double s = strided_sum(part_mu + k * DP + d, npart, (int64_t)KP * DP);
    float* o = mu_acc + j;
    *o = accumulate ? (float)((double)*o + s) : (float)s;
    return;
  }
  const int64_t kk = j - K * D;
  if (kk < K) {
    const double s = strided_sum(part_nk + kk, npart, KP);
    Nk[kk] = accumulate ? (float)((double)Nk[kk] + s) : (float)s;
  }
}

template <int DP>
hipError_t launch_bf16(const FullPlan& pl, const float* X, int64_t ldx, unsigned char* ws, float* logZ,
                       bool run1, bool run2, bool dense, hipStream_t stream) {
  const bf16x8* lop = reinterpret_cast<const bf16x8*>(ws + pl.off_lop);
  const float* bsw = reinterpret_cast<const float*>(ws + pl.off_bsw);
  const float* ck = reinterpret_cast<const float*>(ws + pl.off_ck);
  float* rowstat = reinterpret_cast<float*>(ws + pl.off_rowstat);
  float* lj = reinterpret_cast<float*>(ws + pl.off_lj);
  if (run1) {
    constexpr size_t lds1 = bf16_lse_lds_bytes<DP>();
    if (lds1 > 65536) {
      hipError_t e = hipFuncSetAttribute(reinterpret_cast<const void*>(&full_bf16_lse<DP>),
                                         hipFuncAttributeMaxDynamicSharedMemorySize, (int)lds1);
      if (e != hipSuccess) return e;
    }
    hipLaunchKernelGGL(full_bf16_lse<DP>, dim3((unsigned)cdiv(pl.N, 32 * kWaves)), dim3(kThreads), lds1,
                       stream, X, ldx, pl.N, (int)pl.D, lop, bsw, ck, (int)pl.K, pl.KP, logZ, rowstat, lj);
  }
  if (!run2) return hipGetLastError();
  constexpr size_t lds2 = bf16_accum_lds_bytes<DP>();
  static_assert(lds2 <= (size_t)160 * 1024, "pass-2 tiles fit LDS");
  if (lds2 > 65536) {
    hipError_t e = hipFuncSetAttribute(reinterpret_cast<const void*>(&full_bf16_accum<DP>),
                                       hipFuncAttributeMaxDynamicSharedMemorySize, (int)lds2);
    if (e != hipSuccess) return e;
  }
  hipLaunchKernelGGL(full_bf16_accum<DP>, dim3((unsigned)(pl.nslab * pl.ncg)), dim3(kAccThreads), lds2,
                     stream, X, ldx, pl.N, (int)pl.D, (int)pl.K, pl.KP, rowstat, lj, pl.nslab,
                     pl.rows_per_slab, reinterpret_cast<float*>(ws + pl.off_part_sig),
                     reinterpret_cast<float*>(ws + pl.off_part_mu),
                     reinterpret_cast<float*>(ws + pl.off_part_nk), dense ? 1 : 0);
  return hipGetLastError();
}

}  // namespace
}  // namespace fgmm

using namespace fgmm;

namespace {
// Rows per call of the plans that always store the log-joint (the bf16 contract and
// D > 256), whose N/32 tiles of KP x 32 floats (rounded up to 8) must fit
// kMaxLjBytes: a multiple of 256 rows.  Larger calls run in chunks of this many rows.
bool full_lj_chunked(int64_t D, bool bf16) { return bf16 || full_is_wide((int)round_up(D, 32)); }
int64_t full_lj_chunk_rows(int64_t K) {
  const int64_t KP = round_up(K < 1 ? 1 : K, kCompsPerWG);
  const int64_t tiles = (int64_t)(kMaxLjBytes / ((size_t)KP * 32 * sizeof(float))) / 8 * 8;
  return tiles * 32;
}
}  // namespace

extern "C" size_t fgmm_full_workspace_bytes(int64_t N, int64_t K, int64_t D) {
  return fgmm_full_workspace_bytes_ex(N, K, D, 0u);
}

extern "C" size_t fgmm_full_workspace_bytes_ex(int64_t N, int64_t K, int64_t D, unsigned flags) {
  if (N < 0 || K < 0 || D < 1) return 0;
  const bool bf16 = (flags & FGMM_FLAG_BF16) != 0;
  if (D > (bf16 ? 128 : kFullMaxD)) return 0;
  const int64_t rows = full_lj_chunked(D, bf16) ? std::min(N, full_lj_chunk_rows(K)) : N;
  return make_plan(rows, K, D, wants_stored_lj(flags), bf16, wants_auto_lj(flags)).total;
}

extern "C" int fgmm_full_estep_f32(const float* X, int64_t ldx, int64_t N, int64_t D, const float* mu,
                                   int64_t ldmu, int64_t K, const float* prec_chol, const float* log_pi,
                                   float* logZ, float* Nk, float* mu_acc, float* sig_outer,
                                   void* workspace, size_t workspace_bytes, unsigned flags,
                                   void* stream_) {
  hipStream_t stream = reinterpret_cast<hipStream_t>(stream_);
  const bool want_logz = !(flags & FGMM_FLAG_NO_LOGZ);
  const bool accumulate = (flags & FGMM_FLAG_ACCUMULATE) != 0;
  const bool dense = (flags & FGMM_FLAG_DENSE) != 0;
  if (N < 0 || K < 0 || D < 1) return FGMM_ERR_INVALID_ARG;
  if (N > 0 && (X == nullptr || ldx < round_up(D, 4) || (ldx % 4) != 0 ||
                (reinterpret_cast<uintptr_t>(X) & 15) != 0))
    return FGMM_ERR_INVALID_ARG;
  if (N > 0 && want_logz && logZ == nullptr) return FGMM_ERR_INVALID_ARG;
  if (K > 0 && (mu == nullptr || ldmu < D || prec_chol == nullptr || log_pi == nullptr ||
                Nk == nullptr || mu_acc == nullptr || sig_outer == nullptr))
    return FGMM_ERR_INVALID_ARG;
  if (N > kMaxRows || K > (int64_t)1 << 20) return FGMM_ERR_UNSUPPORTED;
  const bool bf16 = (flags & FGMM_FLAG_BF16) != 0;
  if (D > (bf16 ? 128 : kFullMaxD)) return FGMM_ERR_UNSUPPORTED;
  {
    // Launch grids: the sig_outer finish runs one workgroup per (component, upper block).
    const int64_t nmb = cdiv(D, 32);
    if (K * (nmb * (nmb + 1) / 2) >= ((int64_t)1 << 24)) return FGMM_ERR_UNSUPPORTED;
  }
  if (full_lj_chunked(D, bf16) && K > 0 && N > full_lj_chunk_rows(K)) {
    // The bf16 contract and D > 256 store the log-joint, at most kMaxLjBytes per call:
    // larger N runs as consecutive row chunks on one workspace, each chunk after the
    // first adding its statistics to the outputs.  A phase split cannot span the chunks.
    if (flags & (FGMM_FLAG_PHASE1 | FGMM_FLAG_PHASE2)) return FGMM_ERR_UNSUPPORTED;
    const int64_t rows = full_lj_chunk_rows(K);
    for (int64_t r0 = 0; r0 < N; r0 += rows) {
      const int64_t n = std::min(rows, N - r0);
      const unsigned f = r0 == 0 ? flags : (flags | FGMM_FLAG_ACCUMULATE);
      const int st = fgmm_full_estep_f32(X + r0 * ldx, ldx, n, D, mu, ldmu, K, prec_chol, log_pi,
                                         logZ ? logZ + r0 : nullptr, Nk, mu_acc, sig_outer, workspace,
                                         workspace_bytes, f, stream_);
      if (st != FGMM_OK) return st;
    }
    return FGMM_OK;
  }
  const FullPlan pl = make_plan(N, K, D, wants_stored_lj(flags), bf16, wants_auto_lj(flags) && ldx <= kMaxBufLdx);
  // The bf16 contract always stores the log-joint: N x K floats within kMaxLjBytes.
  if (bf16 && K > 0 && !pl.lj) return FGMM_ERR_UNSUPPORTED;
  if (workspace_bytes < pl.total || (pl.total > 0 && workspace == nullptr)) return FGMM_ERR_WORKSPACE;
  if (!want_logz) logZ = nullptr;
  unsigned char* ws = static_cast<unsigned char*>(workspace);
  const bool sel1 = (flags & FGMM_FLAG_PHASE1) != 0, sel2 = (flags & FGMM_FLAG_PHASE2) != 0;
  const bool run1 = sel1 || !sel2, run2 = sel2 || !sel1;

  if (K == 0) {
    if (N > 0 && logZ)
      hipLaunchKernelGGL(full_fill, dim3((unsigned)cdiv(N, 256)), dim3(256), 0, stream, logZ, N,
                         -INFINITY);
    return hipGetLastError() == hipSuccess ? FGMM_OK : FGMM_ERR_HIP;
  }
  if (run1 && bf16)
    hipLaunchKernelGGL(full_bf16_prep, dim3((unsigned)pl.KP), dim3(64), 0, stream, mu, ldmu, prec_chol, K,
                       (int)D, pl.DP, log_pi, reinterpret_cast<bf16x8*>(ws + pl.off_lop),
                       reinterpret_cast<float*>(ws + pl.off_bsw), reinterpret_cast<float*>(ws + pl.off_ck));
  else if (run1 && pl.wide)
    hipLaunchKernelGGL(full_x6_prep_wide, dim3((unsigned)((int64_t)pl.KP * pl.NMB)), dim3(256), 0, stream, mu,
                       ldmu, prec_chol, K, (int)D, pl.DP, log_pi, reinterpret_cast<bf16x8*>(ws + pl.off_l3),
                       reinterpret_cast<double*>(ws + pl.off_esw), reinterpret_cast<double*>(ws + pl.off_ck));
  else if (run1)
    hipLaunchKernelGGL(full_x6_prep, dim3((unsigned)pl.KP), dim3(256), 0, stream, mu, ldmu, prec_chol, K,
                       (int)D, pl.DP, log_pi, reinterpret_cast<bf16x8*>(ws + pl.off_l3),
                       reinterpret_cast<double*>(ws + pl.off_esw), reinterpret_cast<double*>(ws + pl.off_ck));
  if (N > 0) {
    auto run = [&](auto dp_tag) -> hipError_t {
      constexpr int DP = decltype(dp_tag)::value;
      if constexpr (DP <= 128)
        return bf16 ? launch_bf16<DP>(pl, X, ldx, ws, logZ, run1, run2, dense, stream)
                    : launch_passes<DP>(pl, X, ldx, ws, logZ, run1, run2, dense, stream);
      else
        return launch_passes<DP>(pl, X, ldx, ws, logZ, run1, run2, dense, stream);
    };
    hipError_t e = hipSuccess;
    switch (pl.wide ? 0 : pl.DP) {
      case 0: e = launch_wide(pl, X, ldx, ws, logZ, run1, run2, dense, stream); break;
      case 32: e = run(std::integral_constant<int, 32>{}); break;
      case 64: e = run(std::integral_constant<int, 64>{}); break;
      case 96: e = run(std::integral_constant<int, 96>{}); break;
      case 128: e = run(std::integral_constant<int, 128>{}); break;
      case 160: e = run(std::integral_constant<int, 160>{}); break;
      case 192: e = run(std::integral_constant<int, 192>{}); break;
      case 224: e = run(std::integral_constant<int, 224>{}); break;
      case 256: e = run(std::integral_constant<int, 256>{}); break;
      default: return FGMM_ERR_UNSUPPORTED;
    }
    if (e != hipSuccess) return FGMM_ERR_HIP;
  }
  if (!run2) return hipGetLastError() == hipSuccess ? FGMM_OK : FGMM_ERR_HIP;
  const int64_t nthreads = K * D * D + K * D + K;
  const int64_t nvec = K * D + K;
  const int64_t nsb = (int64_t)pl.NMB * (pl.NMB + 1) / 2;
  if (bf16) {
    hipLaunchKernelGGL(full_bf16_reduce, dim3((unsigned)cdiv(nthreads, 256)), dim3(256), 0, stream,
                       reinterpret_cast<const float*>(ws + pl.off_part_sig),
                       reinterpret_cast<const float*>(ws + pl.off_part_mu),
                       reinterpret_cast<const float*>(ws + pl.off_part_nk), pl.npart, pl.KP, pl.DP,
                       pl.NMB, K, (int)D, Nk, mu_acc, sig_outer, accumulate ? 1 : 0);
    return hipGetLastError() == hipSuccess ? FGMM_OK : FGMM_ERR_HIP;
  }
  if (flags & FGMM_FLAG_ATOMIC_REDUCE) {
    if (!accumulate) {
      hipLaunchKernelGGL(full_fill, dim3((unsigned)cdiv(K, 256)), dim3(256), 0, stream, Nk, K, 0.0f);
      hipLaunchKernelGGL(full_fill, dim3((unsigned)cdiv(K * D, 256)), dim3(256), 0, stream, mu_acc, K * D, 0.0f);
      hipLaunchKernelGGL(full_fill, dim3((unsigned)cdiv(K * D * D, 256)), dim3(256), 0, stream, sig_outer,
                         K * D * D, 0.0f);
    }
    if (pl.npart > 0) {
      hipLaunchKernelGGL(full_reduce_sig<true>, dim3((unsigned)(K * nsb), (unsigned)pl.npart), dim3(256), 0,
                         stream, reinterpret_cast<const float*>(ws + pl.off_part_sig), pl.npart, pl.KP, pl.NMB,
                         (int)D, sig_outer, 1);
      hipLaunchKernelGGL(full_reduce<true>, dim3((unsigned)cdiv(nvec, 256), (unsigned)pl.npart), dim3(256), 0,
                         stream, reinterpret_cast<const float*>(ws + pl.off_part_mu),
                         reinterpret_cast<const float*>(ws + pl.off_part_nk), pl.npart, pl.KP, pl.DP, K,
                         (int)D, Nk, mu_acc, 1);
    }
    return hipGetLastError() == hipSuccess ? FGMM_OK : FGMM_ERR_HIP;
  }
  hipLaunchKernelGGL(full_reduce_sig<false>, dim3((unsigned)(K * nsb)), dim3(256), 0, stream,
                     reinterpret_cast<const float*>(ws + pl.off_part_sig), pl.npart, pl.KP, pl.NMB, (int)D,
                     sig_outer, accumulate ? 1 : 0);
  hipLaunchKernelGGL(full_reduce<false>, dim3((unsigned)cdiv(nvec, 256)), dim3(256), 0, stream,
                     reinterpret_cast<const float*>(ws + pl.off_part_mu),
                     reinterpret_cast<const float*>(ws + pl.off_part_nk), pl.npart, pl.KP, pl.DP, K,
                     (int)D, Nk, mu_acc, accumulate ? 1 : 0);
  return hipGetLastError() == hipSuccess ? FGMM_OK : FGMM_ERR_HIP;
}
