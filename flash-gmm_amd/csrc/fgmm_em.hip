// EM driver pieces: the GPU M-steps (isotropic, diagonal, full covariance), a
// deterministic sum of logZ, and the streaming isotropic EM driver for data sets
// larger than HBM.
//
// M-step (README.md:59-61, :99-100):  pi = Nk / N,  mu = mu_acc / Nk,
// sigma^2 = sig_acc / (D Nk).  sig_acc is accumulated about the previous means, so
// that estimate exceeds the sample variance by ||mu_new - mu_old||^2 / D; the
// FGMM_MSTEP_EXACT_VARIANCE flag removes that term.  Components with Nk = 0 keep
// their mean and variance and get log pi = -inf.
//
// Streaming (README.md:81-103, where each chunk is a synchronous pageable
// chunk.cuda()): rows come from a host row source into two pinned buffers; while
// the host fills one, the other is copied to the device on a copy stream and the
// previous chunk's E-step runs on a compute stream, with events ordering buffer
// reuse.  The E-step accumulates Nk / mu_acc / sig_acc across chunks and the
// M-step runs on the device after the last chunk of each iteration.

#include "fgmm_common.hpp"

#include <math.h>

#include <algorithm>
#include <chrono>
#include <vector>

namespace fgmm {
namespace {

__global__ __launch_bounds__(256) void iso_mstep_kernel(const float* __restrict__ Nk,
                                                        const float* __restrict__ mu_acc,
                                                        const float* __restrict__ sig_acc, double N,
                                                        int D, double var_floor, int exact,
                                                        float* __restrict__ mu, int64_t ldmu,
                                                        float* __restrict__ lss, float* __restrict__ lpi) {
  __shared__ double red[256];
  const int64_t k = blockIdx.x;
  const int t = threadIdx.x;
  const double nk = (double)Nk[k];
  if (!(nk > 0.0)) {
    if (t == 0) lpi[k] = -INFINITY;
    return;
  }
  // Shift of the mean, summed over dimensions (old means read before any write).
  double sh = 0.0;
  for (int d = t; d < D; d += blockDim.x) {
    const double mn = (double)mu_acc[k * D + d] / nk;
    const double dm = mn - (double)mu[k * ldmu + d];
    sh = fma(dm, dm, sh);
  }
  red[t] = sh;
  __syncthreads();
  for (int s = blockDim.x / 2; s > 0; s >>= 1) {
    if (t < s) red[t] += red[t + s];
    __syncthreads();
  }
  for (int d = t; d < D; d += blockDim.x) mu[k * ldmu + d] = (float)((double)mu_acc[k * D + d] / nk);
  if (t == 0) {
    double s2 = (double)sig_acc[k] / ((double)D * nk);
    if (exact) s2 -= red[0] / (double)D;
    if (s2 < var_floor) s2 = var_floor;
    lss[k] = (float)log(s2);
    lpi[k] = (float)log(nk / N);
  }
}

// Diagonal M-step, one block per component: pi, mu and per-dimension variances
// sigma^2_kd = sig_acc_kd / Nk_k (accumulated about the old means; the exact form
// subtracts (mu_new - mu_old)^2).
__global__ __launch_bounds__(256) void diag_mstep_kernel(const float* __restrict__ Nk,
                                                         const float* __restrict__ mu_acc,
                                                         const float* __restrict__ sig_acc, double N,
                                                         int D, double var_floor, int exact,
                                                         float* __restrict__ mu, int64_t ldmu,
                                                         float* __restrict__ lss, int64_t ldlss,
                                                         float* __restrict__ lpi) {
  const int64_t k = blockIdx.x;
  const double nk = (double)Nk[k];
  if (!(nk > 0.0)) {
    if (threadIdx.x == 0) lpi[k] = -INFINITY;
    return;
  }
  for (int d = threadIdx.x; d < D; d += blockDim.x) {
    const double mn = (double)mu_acc[k * D + d] / nk;
    double s2 = (double)sig_acc[k * D + d] / nk;
    if (exact) {
      const double dm = mn - (double)mu[k * ldmu + d];
      s2 -= dm * dm;
    }
    if (s2 < var_floor) s2 = var_floor;
    mu[k * ldmu + d] = (float)mn;
    lss[k * ldlss + d] = (float)log(s2);
  }
  if (threadIdx.x == 0) lpi[k] = (float)log(nk / N);
}

// Full-covariance M-step, one block per component, fp64 in LDS:
//   Sigma = sig_outer / Nk - mu mu^T + reg I,  Sigma = U U^T with U upper-triangular
//   (Cholesky taken from the last column), W = U^-1, and prec_chol = L = W^T, the
//   lower-triangular factor with L L^T = Sigma^-1 and a positive diagonal.
// A pivot that is not positive (Sigma not positive definite) is replaced by the
// ridge (or 1e-30) and counted in *info.
// The full M-step takes D up to this; above D = 128 it works in device scratch of
// at most kMstepScratchBytes (at least one component's two D x D fp64 matrices).
constexpr int kFullMstepMaxD = 4096;
constexpr size_t kMstepScratchBytes = (size_t)1 << 30;

__global__ __launch_bounds__(256) void full_mstep_kernel(const float* __restrict__ Nk,
                                                         const float* __restrict__ mu_acc,
                                                         const float* __restrict__ sig_outer, double N,
                                                         int D, double reg, float* __restrict__ mu,
                                                         int64_t ldmu, float* __restrict__ prec_chol,
                                                         float* __restrict__ lpi, int* __restrict__ info) {
  extern __shared__ double lds_d[];
  double* S = lds_d;            // D x D: U in the upper triangle, W^T below it
  double* m = S + D * D;        // new mean
  double* wd = m + D;           // diagonal of W
  __shared__ double piv;
  const int64_t k = blockIdx.x;
  const int t = threadIdx.x, nt = blockDim.x;
  const double nk = (double)Nk[k];
  if (!(nk > 0.0)) {
    if (t == 0) lpi[k] = -INFINITY;
    return;
  }
  for (int i = t; i < D; i += nt) m[i] = (double)mu_acc[k * D + i] / nk;
  __syncthreads();
  const float* so = sig_outer + k * (int64_t)D * D;
  for (int e = t; e < D * D; e += nt) {
    const int i = e / D, j = e % D;
    double v = 0.5 * ((double)so[i * D + j] + (double)so[j * D + i]) / nk - m[i] * m[j];
    if (i == j) v += reg;
    S[e] = v;
  }
  __syncthreads();
  bool indefinite = false;   // thread 0 only
  for (int j = D - 1; j >= 0; --j) {
    if (t == 0) {
      double d = S[j * D + j];
      if (!(d > 0.0)) {
        d = reg > 0.0 ? reg : 1e-30;
        indefinite = true;
      }
      piv = sqrt(d);
      S[j * D + j] = piv;
    }
    __syncthreads();
    const double p = piv;
    for (int i = t; i < j; i += nt) S[i * D + j] /= p;
    __syncthreads();
    for (int e = t; e < j * j; e += nt) {
      const int a = e / j, b = e % j;
      if (a <= b) S[a * D + b] -= S[a * D + j] * S[b * D + j];
    }
    __syncthreads();
  }
  if (t == 0 && indefinite && info) atomicAdd(info, 1);
  // Column c of W = U^-1 by back substitution, stored transposed in row c below the diagonal.
  for (int c = t; c < D; c += nt) {
    wd[c] = 1.0 / S[c * D + c];
    for (int i = c - 1; i >= 0; --i) {
      double acc = S[i * D + c] * wd[c];
      for (int l = i + 1; l < c; ++l) acc += S[i * D + l] * S[c * D + l];
      S[c * D + i] = -acc / S[i * D + i];
    }
  }
  __syncthreads();
  float* L = prec_chol + k * (int64_t)D * D;
  for (int e = t; e < D * D; e += nt) {
    const int i = e / D, j = e % D;
    L[e] = (float)(j < i ? S[i * D + j] : (j == i ? wd[i] : 0.0));
  }
  for (int i = t; i < D; i += nt) mu[k * ldmu + i] = (float)m[i];
  if (t == 0) lpi[k] = (float)log(nk / N);
}

// The same M-step above D = 128, where the D x D fp64 matrix no longer fits in LDS:
// per component a D x D fp64 matrix S (Sigma, then U in its upper triangle) and a
// D x D fp64 W = U^-1 (row-major) in device scratch, 1024 threads per component.
//   Cholesky from the last column: for j = D-1 .. 0 the pivot, column j of U (kept
//   in LDS), then the update of the leading j x j block's upper triangle;
//   W row by row from the bottom (U W = I): W[i][c] = -(sum_{l=i+1..c} U[i][l] W[l][c])
//   / U[i][i], the threads over c reading row i of U from LDS and rows of W coalesced;
//   prec_chol = W^T.
__global__ __launch_bounds__(1024) void full_mstep_wide_kernel(const float* __restrict__ Nk,
                                                               const float* __restrict__ mu_acc,
                                                               const float* __restrict__ sig_outer, double N,
                                                               int D, double reg, float* __restrict__ mu,
                                                               int64_t ldmu, float* __restrict__ prec_chol,
                                                               float* __restrict__ lpi, int* __restrict__ info,
                                                               int64_t k0, double* __restrict__ scratch) {
  extern __shared__ double lds_d[];
  double* col = lds_d;        // column j (Cholesky) or row i (inverse) of U
  double* m = col + D;        // new mean
  __shared__ double piv;
  const int64_t k = k0 + blockIdx.x;
  const int t = threadIdx.x, nt = blockDim.x;
  const int64_t DD = (int64_t)D * D;
  double* S = scratch + (int64_t)blockIdx.x * 2 * DD;
  double* W = S + DD;
  const double nk = (double)Nk[k];
  if (!(nk > 0.0)) {
    if (t == 0) lpi[k] = -INFINITY;
    return;
  }
  for (int i = t; i < D; i += nt) m[i] = (double)mu_acc[k * D + i] / nk;
  __syncthreads();
  const float* so = sig_outer + k * DD;
  for (int64_t e = t; e < DD; e += nt) {
    const int i = (int)(e / D), j = (int)(e % D);
    double v = 0.5 * ((double)so[e] + (double)so[(int64_t)j * D + i]) / nk - m[i] * m[j];
    if (i == j) v += reg;
    S[e] = v;
  }
  __syncthreads();
  bool indefinite = false;   // thread 0 only
  for (int j = D - 1; j >= 0; --j) {
    if (t == 0) {
      double d = S[(int64_t)j * D + j];
      if (!(d > 0.0)) {
        d = reg > 0.0 ? reg : 1e-30;
        indefinite = true;
      }
      piv = sqrt(d);
      S[(int64_t)j * D + j] = piv;
    }
    __syncthreads();
    const double p = piv;
    for (int i = t; i < j; i += nt) {
      const double v = S[(int64_t)i * D + j] / p;
      S[(int64_t)i * D + j] = v;
      col[i] = v;
    }
    __syncthreads();
    // Upper triangle of the leading j x j block: row a, columns a .. j - 1.
    for (int64_t e = t; e < (int64_t)j * j; e += nt) {
      const int a = (int)(e / j), b = (int)(e % j);
      if (a <= b) S[(int64_t)a * D + b] -= col[a] * col[b];
    }
    __syncthreads();
  }
  if (t == 0 && indefinite && info) atomicAdd(info, 1);
  for (int i = D - 1; i >= 0; --i) {
    for (int l = i + t; l < D; l += nt) col[l] = S[(int64_t)i * D + l];
    __syncthreads();
    const double uii = col[i];
    for (int c = i + t; c < D; c += nt) {
      double acc = 0.0;
      for (int l = i + 1; l <= c; ++l) acc = fma(col[l], W[(int64_t)l * D + c], acc);
      W[(int64_t)i * D + c] = c == i ? 1.0 / uii : -acc / uii;
    }
    __syncthreads();
  }
  float* L = prec_chol + k * DD;
  for (int64_t e = t; e < DD; e += nt) {
    const int i = (int)(e / D), j = (int)(e % D);
    L[e] = (float)(j <= i ? W[(int64_t)j * D + i] : 0.0);
  }
  for (int i = t; i < D; i += nt) mu[k * ldmu + i] = (float)m[i];
  if (t == 0) lpi[k] = (float)log(nk / N);
}

// Deterministic sum of n floats into *acc (fp64): fixed 1024-element blocks, then
// the block sums by one workgroup in a fixed order (sum_parts).
__global__ __launch_bounds__(256) void sum_blocks(const float* __restrict__ x, int64_t n,
                                                  double* __restrict__ part) {
  __shared__ double red[256];
  const int64_t base = (int64_t)blockIdx.x * 1024;
  double s = 0.0;
  for (int i = threadIdx.x; i < 1024; i += 256) {
    const int64_t j = base + i;
    if (j < n) s += (double)x[j];
  }
  red[threadIdx.x] = s;
  __syncthreads();
  for (int st = 128; st > 0; st >>= 1) {
    if (threadIdx.x < st) red[threadIdx.x] += red[threadIdx.x + st];
    __syncthreads();
  }
  if (threadIdx.x == 0) part[blockIdx.x] = red[0];
}

// One 256-thread workgroup: thread t adds parts t, t + 256, ... in order, then a
// fixed tree over the threads (deterministic; 16K parts per 16M-row chunk took
// 0.94 ms on one thread).
__global__ __launch_bounds__(256) void sum_parts(const double* __restrict__ part, int64_t nparts,
                                                 double* __restrict__ acc) {
  __shared__ double red[256];
  double s = 0.0;
  for (int64_t i = threadIdx.x; i < nparts; i += 256) s += part[i];
  red[threadIdx.x] = s;
  __syncthreads();
  for (int st = 128; st > 0; st >>= 1) {
    if (threadIdx.x < st) red[threadIdx.x] += red[threadIdx.x + st];
    __syncthreads();
  }
  if (threadIdx.x == 0) *acc += red[0];
}

__global__ __launch_bounds__(256) void fill_f32(float* __restrict__ p, int64_t n, float v) {
  const int64_t i = (int64_t)blockIdx.x * blockDim.x + threadIdx.x;
  if (i < n) p[i] = v;
}

__global__ void fill_f64_one(double* p, double v) {
  if (threadIdx.x == 0 && blockIdx.x == 0) *p = v;
}

double ms_since(std::chrono::steady_clock::time_point t0) {
  return std::chrono::duration<double, std::milli>(std::chrono::steady_clock::now() - t0).count();
}

// Owner of every resource the streaming driver creates; releases them in any exit path.
struct StreamRes {
  float* pinned[2] = {nullptr, nullptr};
  float* dev[2] = {nullptr, nullptr};
  void* ws = nullptr;
  float *Nk = nullptr, *mu_acc = nullptr, *sig_acc = nullptr, *logZ = nullptr;
  double *part = nullptr, *ll = nullptr;
  hipStream_t copy = nullptr, comp = nullptr;
  hipEvent_t h2d0[2] = {nullptr, nullptr}, h2d1[2] = {nullptr, nullptr};
  hipEvent_t e0[2] = {nullptr, nullptr}, e1[2] = {nullptr, nullptr};
  std::vector<hipEvent_t> m0, m1;  // per iteration, around the M-step
  ~StreamRes() {
    if (comp) (void)hipStreamSynchronize(comp);
    if (copy) (void)hipStreamSynchronize(copy);
    for (int b = 0; b < 2; ++b) {
      if (pinned[b]) (void)hipHostFree(pinned[b]);
      if (dev[b]) (void)hipFree(dev[b]);
      for (hipEvent_t e : {h2d0[b], h2d1[b], e0[b], e1[b]})
        if (e) (void)hipEventDestroy(e);
    }
    for (void* p : {(void*)ws, (void*)Nk, (void*)mu_acc, (void*)sig_acc, (void*)logZ, (void*)part, (void*)ll})
      if (p) (void)hipFree(p);
    for (hipEvent_t e : m0)
      if (e) (void)hipEventDestroy(e);
    for (hipEvent_t e : m1)
      if (e) (void)hipEventDestroy(e);
    if (copy) (void)hipStreamDestroy(copy);
    if (comp) (void)hipStreamDestroy(comp);
  }
};

}  // namespace
}  // namespace fgmm

using namespace fgmm;

extern "C" int fgmm_iso_mstep_f32(const float* Nk, const float* mu_acc, const float* sig_acc, int64_t N,
                                  int64_t K, int64_t D, double var_floor, float* mu, int64_t ldmu,
                                  float* log_sigma_sq, float* log_pi, unsigned flags, void* stream) {
  if (N < 0 || K < 0 || D < 1 || ldmu < D || !(var_floor >= 0.0)) return FGMM_ERR_INVALID_ARG;
  if (K == 0) return FGMM_OK;
  if (!Nk || !mu_acc || !sig_acc || !mu || !log_sigma_sq || !log_pi) return FGMM_ERR_INVALID_ARG;
  hipLaunchKernelGGL(iso_mstep_kernel, dim3((unsigned)K), dim3(256), 0, (hipStream_t)stream, Nk,
                     mu_acc, sig_acc, (double)N, (int)D, var_floor,
                     (flags & FGMM_MSTEP_EXACT_VARIANCE) ? 1 : 0, mu, ldmu, log_sigma_sq, log_pi);
  return hipGetLastError() == hipSuccess ? FGMM_OK : FGMM_ERR_HIP;
}

extern "C" int fgmm_diag_mstep_f32(const float* Nk, const float* mu_acc, const float* sig_acc, int64_t N,
                                   int64_t K, int64_t D, double var_floor, float* mu, int64_t ldmu,
                                   float* log_sigma_sq, int64_t ldlss, float* log_pi, unsigned flags,
                                   void* stream) {
  if (N < 0 || K < 0 || D < 1 || ldmu < D || ldlss < D || !(var_floor >= 0.0)) return FGMM_ERR_INVALID_ARG;
  if (K == 0) return FGMM_OK;
  if (!Nk || !mu_acc || !sig_acc || !mu || !log_sigma_sq || !log_pi) return FGMM_ERR_INVALID_ARG;
  hipLaunchKernelGGL(diag_mstep_kernel, dim3((unsigned)K), dim3(256), 0, (hipStream_t)stream, Nk,
                     mu_acc, sig_acc, (double)N, (int)D, var_floor,
                     (flags & FGMM_MSTEP_EXACT_VARIANCE) ? 1 : 0, mu, ldmu, log_sigma_sq, ldlss, log_pi);
  return hipGetLastError() == hipSuccess ? FGMM_OK : FGMM_ERR_HIP;
}

extern "C" int fgmm_full_mstep_f32(const float* Nk, const float* mu_acc, const float* sig_outer, int64_t N,
                                   int64_t K, int64_t D, double reg_covar, float* mu, int64_t ldmu,
                                   float* prec_chol, float* log_pi, int* info, void* stream) {
  if (N < 0 || K < 0 || D < 1 || ldmu < D || !(reg_covar >= 0.0)) return FGMM_ERR_INVALID_ARG;
  if (D > kFullMstepMaxD) return FGMM_ERR_UNSUPPORTED;
  if (K == 0) return FGMM_OK;
  if (!Nk || !mu_acc || !sig_outer || !mu || !prec_chol || !log_pi) return FGMM_ERR_INVALID_ARG;
  if (D > 128) {
    // Components in batches whose two D x D fp64 matrices fit kMstepScratchBytes,
    // on scratch allocated and freed in stream order.
    const size_t per = (size_t)2 * (size_t)D * (size_t)D * sizeof(double);
    const int64_t batch = std::max<int64_t>(1, std::min<int64_t>(K, (int64_t)(kMstepScratchBytes / per)));
    void* scratch = nullptr;
    if (hipMallocAsync(&scratch, per * (size_t)batch, (hipStream_t)stream) != hipSuccess) return FGMM_ERR_HIP;
    const size_t lds = (size_t)2 * D * sizeof(double);
    if (lds > 32768) {
      const hipError_t e = hipFuncSetAttribute(reinterpret_cast<const void*>(&full_mstep_wide_kernel),
                                               hipFuncAttributeMaxDynamicSharedMemorySize, (int)lds);
      if (e != hipSuccess) {
        (void)hipFreeAsync(scratch, (hipStream_t)stream);
        return FGMM_ERR_HIP;
      }
    }
    for (int64_t k0 = 0; k0 < K; k0 += batch) {
      const int64_t nb = std::min(batch, K - k0);
      hipLaunchKernelGGL(full_mstep_wide_kernel, dim3((unsigned)nb), dim3(1024), lds, (hipStream_t)stream, Nk,
                         mu_acc, sig_outer, (double)N, (int)D, reg_covar, mu, ldmu, prec_chol, log_pi, info, k0,
                         static_cast<double*>(scratch));
    }
    const hipError_t le = hipGetLastError();
    const hipError_t fe = hipFreeAsync(scratch, (hipStream_t)stream);
    return le == hipSuccess && fe == hipSuccess ? FGMM_OK : FGMM_ERR_HIP;
  }
  const size_t lds = ((size_t)D * D + 2 * (size_t)D) * sizeof(double);
  if (lds > 65536) {
    hipError_t e = hipFuncSetAttribute(reinterpret_cast<const void*>(&full_mstep_kernel),
                                       hipFuncAttributeMaxDynamicSharedMemorySize, (int)lds);
    if (e != hipSuccess) return FGMM_ERR_HIP;
  }
  hipLaunchKernelGGL(full_mstep_kernel, dim3((unsigned)K), dim3(256), lds, (hipStream_t)stream, Nk,
                     mu_acc, sig_outer, (double)N, (int)D, reg_covar, mu, ldmu, prec_chol, log_pi, info);
  return hipGetLastError() == hipSuccess ? FGMM_OK : FGMM_ERR_HIP;
}

extern "C" int fgmm_stream_em_iso(const fgmm_em_config* cfg, fgmm_row_source_fn src, void* user,
                                  float* mu, float* log_sigma_sq, float* log_pi,
                                  fgmm_em_report* report) {
  const auto t_start = std::chrono::steady_clock::now();
  if (!cfg || !src || !mu || !log_sigma_sq || !log_pi) return FGMM_ERR_INVALID_ARG;
  const int64_t N = cfg->N, K = cfg->K, D = cfg->D, R = cfg->chunk_rows;
  const int iters = cfg->iterations;
  if (N < 1 || K < 1 || D < 1 || R < 1 || iters < 0 || !(cfg->var_floor >= 0.0))
    return FGMM_ERR_INVALID_ARG;
  fgmm_em_report rep{};
  const int64_t ld = round_up(D, 4);
  const int64_t rows = R < N ? R : N;
  const size_t chunk_bytes = (size_t)rows * ld * sizeof(float);
  // The E-steps hide behind host generation and copies: keep the lean workspace.
  constexpr unsigned estep_flags = FGMM_FLAG_ACCUMULATE | FGMM_FLAG_RECOMPUTE;
  const size_t ws_bytes = fgmm_iso_workspace_bytes_ex(rows, K, D, estep_flags);
  const int64_t nparts = cdiv(rows, 1024);

  StreamRes res;
  auto ok = [](hipError_t e) { return e == hipSuccess; };
  if (!ok(hipStreamCreateWithFlags(&res.copy, hipStreamNonBlocking)) ||
      !ok(hipStreamCreateWithFlags(&res.comp, hipStreamNonBlocking)))
    return FGMM_ERR_HIP;
  for (int b = 0; b < 2; ++b) {
    if (!ok(hipHostMalloc((void**)&res.pinned[b], chunk_bytes, hipHostMallocDefault)) ||
        !ok(hipMalloc((void**)&res.dev[b], chunk_bytes)) || !ok(hipEventCreate(&res.h2d0[b])) ||
        !ok(hipEventCreate(&res.h2d1[b])) || !ok(hipEventCreate(&res.e0[b])) ||
        !ok(hipEventCreate(&res.e1[b])))
      return FGMM_ERR_HIP;
  }
  const int nll = iters > 0 ? iters : 1;
  if (!ok(hipMalloc(&res.ws, ws_bytes > 0 ? ws_bytes : 256)) ||
      !ok(hipMalloc((void**)&res.Nk, K * sizeof(float))) ||
      !ok(hipMalloc((void**)&res.mu_acc, K * D * sizeof(float))) ||
      !ok(hipMalloc((void**)&res.sig_acc, K * sizeof(float))) ||
      !ok(hipMalloc((void**)&res.logZ, rows * sizeof(float))) ||
      !ok(hipMalloc((void**)&res.part, nparts * sizeof(double))) ||
      !ok(hipMalloc((void**)&res.ll, nll * sizeof(double))))
    return FGMM_ERR_HIP;
  res.m0.assign(iters, nullptr);
  res.m1.assign(iters, nullptr);
  for (int it = 0; it < iters; ++it)
    if (!ok(hipEventCreate(&res.m0[it])) || !ok(hipEventCreate(&res.m1[it]))) return FGMM_ERR_HIP;
  rep.device_bytes = 2 * chunk_bytes + ws_bytes + (size_t)K * (D + 2) * sizeof(float) +
                     (size_t)rows * sizeof(float) + (size_t)nparts * sizeof(double) +
                     (size_t)nll * sizeof(double);
  rep.pinned_bytes = 2 * chunk_bytes;
  rep.setup_ms = ms_since(t_start);

  const int64_t nchunks = cdiv(N, R);
  // pinned[b] may be refilled once its copy has finished; dev[b] once the E-step
  // that read it has finished (the copy stream waits for that on the device).
  bool copy_pending[2] = {false, false}, estep_pending[2] = {false, false};
  auto drain_copy = [&](int b) -> int {
    if (!copy_pending[b]) return FGMM_OK;
    float a = 0.0f;
    if (!ok(hipEventSynchronize(res.h2d1[b])) || !ok(hipEventElapsedTime(&a, res.h2d0[b], res.h2d1[b])))
      return FGMM_ERR_HIP;
    rep.h2d_ms += a;
    copy_pending[b] = false;
    return FGMM_OK;
  };
  auto drain_estep = [&](int b) -> int {
    if (!estep_pending[b]) return FGMM_OK;
    float e = 0.0f;
    if (!ok(hipEventSynchronize(res.e1[b])) || !ok(hipEventElapsedTime(&e, res.e0[b], res.e1[b])))
      return FGMM_ERR_HIP;
    rep.estep_ms += e;
    estep_pending[b] = false;
    return FGMM_OK;
  };

  // One flat pipeline over (iteration, chunk).  The rows do not depend on the
  // parameters, so the host fills and copies the next iteration's first chunks
  // while the device finishes the last E-steps and the M-step; stream order on
  // the compute stream puts each M-step before the next iteration's E-steps.
  const int64_t total = nchunks * iters;
  for (int64_t g = 0; g < total; ++g) {
    const int it = (int)(g / nchunks);
    const int64_t c = g % nchunks;
    const int b = (int)(g & 1);
    const int64_t row0 = c * R;
    const int64_t n = (row0 + R <= N) ? R : N - row0;
    // The host buffer is free once the copy of the chunk two back has finished.
    int st = drain_copy(b);
    if (st != FGMM_OK) return st;
    const auto tg = std::chrono::steady_clock::now();
    float* host = res.pinned[b];
    st = src(user, row0, n, D, host);
    if (st == 0 && ld != D) {
      // Sources write rows of stride D; the kernels read stride round_up(D, 4).
      for (int64_t r = n - 1; r >= 0; --r)
        for (int64_t d = D - 1; d >= 0; --d) host[r * ld + d] = host[r * D + d];
    }
    rep.source_ms += ms_since(tg);
    if (st != 0) return FGMM_ERR_SOURCE;
    // dev[b] is reused: the copy waits (on the device) for the E-step that read it
    // two chunks back.  Waiting here, and not right after that E-step was queued,
    // keeps the copy of the chunk in between free to overlap that E-step.
    if (estep_pending[b] && !ok(hipStreamWaitEvent(res.copy, res.e1[b], 0))) return FGMM_ERR_HIP;
    if (!ok(hipEventRecord(res.h2d0[b], res.copy)) ||
        !ok(hipMemcpyAsync(res.dev[b], host, (size_t)n * ld * sizeof(float), hipMemcpyHostToDevice,
                           res.copy)) ||
        !ok(hipEventRecord(res.h2d1[b], res.copy)))
      return FGMM_ERR_HIP;
    if (c == 0) {
      hipLaunchKernelGGL(fill_f32, dim3((unsigned)cdiv(K, 256)), dim3(256), 0, res.comp, res.Nk, K, 0.0f);
      hipLaunchKernelGGL(fill_f32, dim3((unsigned)cdiv(K * D, 256)), dim3(256), 0, res.comp, res.mu_acc,
                         K * D, 0.0f);
      hipLaunchKernelGGL(fill_f32, dim3((unsigned)cdiv(K, 256)), dim3(256), 0, res.comp, res.sig_acc, K,
                         0.0f);
      hipLaunchKernelGGL(fill_f64_one, dim3(1), dim3(64), 0, res.comp, res.ll + it, 0.0);
    }
    // Read the timing of the E-step two chunks back before its events are reused
    // (long finished by now: the host has generated a whole chunk since).
    st = drain_estep(b);
    if (st != FGMM_OK) return st;
    if (!ok(hipStreamWaitEvent(res.comp, res.h2d1[b], 0)) || !ok(hipEventRecord(res.e0[b], res.comp)))
      return FGMM_ERR_HIP;
    st = fgmm_iso_estep_f32(res.dev[b], ld, n, D, mu, D, K, log_sigma_sq, log_pi, res.logZ, res.Nk,
                            res.mu_acc, res.sig_acc, res.ws, ws_bytes, estep_flags, res.comp);
    if (st != FGMM_OK) return st;
    hipLaunchKernelGGL(sum_blocks, dim3((unsigned)cdiv(n, 1024)), dim3(256), 0, res.comp, res.logZ, n,
                       res.part);
    hipLaunchKernelGGL(sum_parts, dim3(1), dim3(256), 0, res.comp, res.part, cdiv(n, 1024), res.ll + it);
    if (!ok(hipEventRecord(res.e1[b], res.comp))) return FGMM_ERR_HIP;
    copy_pending[b] = true;
    estep_pending[b] = true;
    if (c == nchunks - 1) {
      if (!ok(hipEventRecord(res.m0[it], res.comp))) return FGMM_ERR_HIP;
      st = fgmm_iso_mstep_f32(res.Nk, res.mu_acc, res.sig_acc, N, K, D, cfg->var_floor, mu, D,
                              log_sigma_sq, log_pi, cfg->mstep_flags, res.comp);
      if (st != FGMM_OK) return st;
      if (!ok(hipEventRecord(res.m1[it], res.comp))) return FGMM_ERR_HIP;
    }
  }
  for (int b = 0; b < 2; ++b) {
    int st = drain_copy(b);
    if (st == FGMM_OK) st = drain_estep(b);
    if (st != FGMM_OK) return st;
  }
  // The last M-step follows the last E-step's event on the compute stream, and both
  // streams are non-blocking (the null-stream copy below does not wait for them):
  // wait for the compute stream before reading its results and events.
  if (!ok(hipStreamSynchronize(res.comp))) return FGMM_ERR_HIP;
  std::vector<double> ll(nll, 0.0);
  if (iters > 0 && !ok(hipMemcpy(ll.data(), res.ll, iters * sizeof(double), hipMemcpyDeviceToHost)))
    return FGMM_ERR_HIP;
  for (int it = 0; it < iters; ++it) {
    float mm = 0.0f;
    if (!ok(hipEventElapsedTime(&mm, res.m0[it], res.m1[it]))) return FGMM_ERR_HIP;
    rep.mstep_ms += mm;
    if (it < FGMM_EM_MAX_REPORTED_ITERS) rep.loglik[it] = ll[it];
  }
  if (!ok(hipGetLastError())) return FGMM_ERR_HIP;
  rep.total_ms = ms_since(t_start);
  rep.iterations = iters;
  if (report) *report = rep;
  return FGMM_OK;
}
