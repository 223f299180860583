/*
 * flashgmm.h -- C ABI of the MI355X (gfx950) Flash-GMM E-step library.
 *
 * Plain pointers and sizes only.  Every pointer argument except `workspace`
 * bookkeeping is a device pointer on the current HIP device; every call is
 * asynchronous on `stream` (a hipStream_t passed as void*, NULL = the null
 * stream) and never synchronises the device.  Functions return FGMM_OK (0) or
 * a negative status; fgmm_strerror() names it.  Nothing aborts or exits.
 *
 * All device memory is owned by the caller: outputs, and a workspace sized by
 * the matching *_workspace_bytes() query.  The library keeps no allocations
 * between calls.  Calls are re-entrant given distinct outputs and workspaces.
 *
 * Layout conventions (row-major, float32):
 *   X      N x D, row stride ldx (elements), unit column stride.  Requires
 *          ldx % 4 == 0, ldx >= round_up(D, 4) and a 16-byte aligned base.
 *   mu     K x D, row stride ldmu, unit column stride (any alignment).
 *   outputs are dense: logZ (N), Nk (K), mu_acc (K x D), sig_acc (K) or
 *   (K x D), sig_outer (K x D x D).
 */
#ifndef FLASHGMM_H
#define FLASHGMM_H

#include <stddef.h>
#include <stdint.h>

#ifdef __cplusplus
extern "C" {
#endif

enum fgmm_status {
    FGMM_OK = 0,
    FGMM_ERR_INVALID_ARG = -1, /* bad shape, stride, alignment or null pointer */
    FGMM_ERR_UNSUPPORTED = -2, /* shape outside the compiled range (e.g. D > 256) */
    FGMM_ERR_WORKSPACE = -3,   /* workspace smaller than *_workspace_bytes() */
    FGMM_ERR_HIP = -4,         /* a HIP runtime call or kernel launch failed */
};

/* Flags (bitwise OR). */
enum fgmm_flags {
    /* Add the new statistics into Nk / mu_acc / sig_acc instead of overwriting
     * them (streaming over row chunks, README.md:86-96). */
    FGMM_FLAG_ACCUMULATE = 1u << 0,
    /* Do not write logZ; the logZ pointer may be NULL.  logZ is still formed
     * internally for the responsibilities. */
    FGMM_FLAG_NO_LOGZ = 1u << 1,
    /* Finish the per-workgroup partials with float atomics instead of the
     * deterministic fixed-order reduction (results then vary in the last
     * bits from run to run). */
    FGMM_FLAG_ATOMIC_REDUCE = 1u << 2,
    /* Phase selection.  Neither bit set = both phases (the whole E-step).
     * PHASE1 alone runs the constant prologue and the log-normaliser pass:
     * it writes logZ (the per-sample log-likelihood, like score_samples) and
     * leaves per-row state in the workspace.  PHASE2 alone runs the
     * accumulation and reduction and requires a workspace filled by a PHASE1
     * call with the same inputs on the same stream. */
    FGMM_FLAG_PHASE1 = 1u << 3,
    FGMM_FLAG_PHASE2 = 1u << 4,
};

/* Library version as MAJOR*10000 + MINOR*100 + PATCH. */
int fgmm_version(void);

/* Static string naming a status code. */
const char *fgmm_strerror(int status);

/* ------------------------------------------------------------------------ */
/* Isotropic (spherical) E-step.                                             */
/* Replaces flash_gmm_estep(X, mu, log_sigma_sq, log_pi, BLOCK_N, BLOCK_K,    */
/* BLOCK_D) at flash_gmm.py:173-217 (and the same-named 4-argument entry of   */
/* flash_gmm_h100.py:254-328):                                                */
/*   logZ_n  = logsumexp_k [ log_pi_k - 0.5*||x_n - mu_k||^2 * exp(-lss_k)    */
/*                           - 0.5*D*(log(2 pi) + lss_k) ]                    */
/*   Nk_k    = sum_n r_nk,  r_nk = exp(ll_nk - logZ_n)                        */
/*   mu_acc  = sum_n r_nk x_n                                                 */
/*   sig_acc = sum_n r_nk ||x_n - mu_k||^2                                    */
/* log_sigma_sq and log_pi are contiguous (K).                                */
/* ------------------------------------------------------------------------ */
size_t fgmm_iso_workspace_bytes(int64_t N, int64_t K, int64_t D);

int fgmm_iso_estep_f32(const float *X, int64_t ldx, int64_t N, int64_t D,
                       const float *mu, int64_t ldmu, int64_t K,
                       const float *log_sigma_sq, const float *log_pi,
                       float *logZ, float *Nk, float *mu_acc, float *sig_acc,
                       void *workspace, size_t workspace_bytes,
                       unsigned flags, void *stream);

/* ------------------------------------------------------------------------ */
/* Diagonal-covariance E-step.                                               */
/* Replaces flash_gmm_estep_diag(X, mu, log_sigma_sq, log_pi) at             */
/* flash_gmm_diag_h100.py:305-384.  log_sigma_sq is K x D with row stride     */
/* ldlss; sig_acc is K x D:                                                   */
/*   ll_nk      = log_pi_k - 0.5*(D log(2 pi) + sum_d lss_kd)                 */
/*                - 0.5 * sum_d (x_nd - mu_kd)^2 exp(-lss_kd)                 */
/*   sig_acc_kd = sum_n r_nk (x_nd - mu_kd)^2                                 */
/* Supports 1 <= D <= 128.                                                    */
/* ------------------------------------------------------------------------ */
size_t fgmm_diag_workspace_bytes(int64_t N, int64_t K, int64_t D);

int fgmm_diag_estep_f32(const float *X, int64_t ldx, int64_t N, int64_t D,
                        const float *mu, int64_t ldmu, int64_t K,
                        const float *log_sigma_sq, int64_t ldlss, const float *log_pi,
                        float *logZ, float *Nk, float *mu_acc, float *sig_acc,
                        void *workspace, size_t workspace_bytes,
                        unsigned flags, void *stream);

/* ------------------------------------------------------------------------ */
/* Full-covariance E-step.                                                   */
/* Replaces flash_gmm_estep_full(X, mu, prec_chol, log_pi) at                */
/* flash_gmm_full_h100.py:235-336.  prec_chol is K x D x D contiguous, each   */
/* L_k lower-triangular with L_k L_k^T = Sigma_k^-1; sig_outer is K x D x D:  */
/*   ll_nk = log_pi_k + sum_d log(|L_k,dd| + 1e-30) - 0.5 D log(2 pi)         */
/*           - 0.5 ||L_k^T (x_n - mu_k)||^2                                   */
/*   sig_outer_k = sum_n r_nk x_n x_n^T   (uncentred second moment)           */
/* Supports 1 <= D <= 64.                                                     */
/* ------------------------------------------------------------------------ */
size_t fgmm_full_workspace_bytes(int64_t N, int64_t K, int64_t D);

int fgmm_full_estep_f32(const float *X, int64_t ldx, int64_t N, int64_t D,
                        const float *mu, int64_t ldmu, int64_t K,
                        const float *prec_chol, const float *log_pi,
                        float *logZ, float *Nk, float *mu_acc, float *sig_outer,
                        void *workspace, size_t workspace_bytes,
                        unsigned flags, void *stream);

#ifdef __cplusplus
}
#endif

#endif /* FLASHGMM_H */
