// fgmm_iso_estep_f32_noalloc: the isotropic E-step with its workspace in a fixed
// device array instead of caller memory, for callers that cannot allocate device
// memory (code under HIP graph capture, tight serving loops).  It has no counterpart
// in the reference.
//
// The array lives in this translation unit's own code object, which holds nothing
// else: a GPU reserves it when this code object is loaded there, which HIP does on
// first use (the first noalloc call's symbol lookup), not when the isotropic kernels
// are first launched.

#include <hip/hip_runtime.h>

#include <mutex>

#include "flashgmm.h"

// Workspace of fgmm_iso_estep_f32_noalloc: one array per GPU.  Host code never passes
// the name `scratch` itself (on the host it is a stand-in, not a device address): the
// device address comes from hipGetSymbolAddress, looked up once per device.
static __device__ __align__(256) unsigned char scratch[FGMM_NOALLOC_SCRATCH_BYTES];

namespace {
constexpr int kMaxScratchDevices = 64;
std::mutex scratch_mutex;
void* scratch_ptr[kMaxScratchDevices];

// Device address of the current device's scratch array (nullptr and a status on error).
int current_scratch(void** out) {
  int dev = 0;
  if (hipGetDevice(&dev) != hipSuccess || dev < 0 || dev >= kMaxScratchDevices) return FGMM_ERR_HIP;
  std::lock_guard<std::mutex> lock(scratch_mutex);
  if (scratch_ptr[dev] == nullptr) {
    void* p = nullptr;
    if (hipGetSymbolAddress(&p, HIP_SYMBOL(scratch)) != hipSuccess || p == nullptr) return FGMM_ERR_HIP;
    scratch_ptr[dev] = p;
  }
  *out = scratch_ptr[dev];
  return FGMM_OK;
}
}  // namespace

namespace {
bool fits(int64_t n, int64_t K, int64_t D, unsigned flags) {
  return fgmm_iso_workspace_bytes_ex(n, K, D, flags) <= FGMM_NOALLOC_SCRATCH_BYTES;
}
}  // namespace

extern "C" int fgmm_iso_estep_f32_noalloc(const float* X, int64_t ldx, int64_t N, int64_t D, const float* mu,
                                          int64_t ldmu, int64_t K, const float* log_sigma_sq,
                                          const float* log_pi, float* logZ, float* Nk, float* mu_acc,
                                          float* sig_acc, unsigned flags, void* stream) {
  if (flags & FGMM_FLAG_STORE_LOGJOINT) return FGMM_ERR_INVALID_ARG;
  if (N < 0 || K < 0 || D < 1) return FGMM_ERR_INVALID_ARG;
  if (fits(N, K, D, flags)) {
    void* ws = nullptr;
    const int st = current_scratch(&ws);
    if (st != FGMM_OK) return st;
    return fgmm_iso_estep_f32(X, ldx, N, D, mu, ldmu, K, log_sigma_sq, log_pi, logZ, Nk, mu_acc, sig_acc, ws,
                              FGMM_NOALLOC_SCRATCH_BYTES, flags, stream);
  }
  // Too many rows for one call's workspace: consecutive row chunks of the largest
  // multiple of 256 rows that fits, on the same scratch and stream, each chunk after
  // the first adding its statistics to the outputs.  A phase split cannot span them.
  if (flags & (FGMM_FLAG_PHASE1 | FGMM_FLAG_PHASE2)) return FGMM_ERR_SCRATCH;
  int64_t lo = 0, hi = N / 256;   // fits(256 lo) holds (lo = 0: nothing yet), fits(256 (hi + 1)) fails
  while (lo < hi) {
    const int64_t mid = (lo + hi + 1) / 2;
    if (fits(256 * mid, K, D, flags)) lo = mid; else hi = mid - 1;
  }
  const int64_t rows = 256 * lo;
  if (rows == 0) return FGMM_ERR_SCRATCH;   // not even 256 rows fit (K and D too large)
  if (X == nullptr || ldx < D) return FGMM_ERR_INVALID_ARG;
  void* ws = nullptr;
  const int st0 = current_scratch(&ws);
  if (st0 != FGMM_OK) return st0;
  for (int64_t r0 = 0; r0 < N; r0 += rows) {
    const int64_t n = N - r0 < rows ? N - r0 : rows;
    if (!fits(n, K, D, flags)) return FGMM_ERR_SCRATCH;
    const unsigned f = r0 == 0 ? flags : (flags | FGMM_FLAG_ACCUMULATE);
    const int st = fgmm_iso_estep_f32(X + r0 * ldx, ldx, n, D, mu, ldmu, K, log_sigma_sq, log_pi,
                                      logZ ? logZ + r0 : nullptr, Nk, mu_acc, sig_acc, ws,
                                      FGMM_NOALLOC_SCRATCH_BYTES, f, stream);
    if (st != FGMM_OK) return st;
  }
  return FGMM_OK;
}
