/*
 * flashgmm.h -- C ABI of the MI355X (gfx950) Flash-GMM E-step library.
 *
 * Plain pointers and sizes only.  Every pointer argument except `workspace`
 * bookkeeping is a device pointer on the current HIP device; every call is
 * asynchronous on `stream` (a hipStream_t passed as void*, NULL = the null
 * stream) and never synchronises the device.  Functions return FGMM_OK (0) or
 * a negative status; fgmm_strerror() names it.  Nothing aborts or exits.
 *
 * All device memory of the E-steps is owned by the caller: outputs, and a
 * workspace sized by the matching *_workspace_bytes() query (fgmm_full_mstep_f32
 * above D = 128 and the streaming driver allocate their own scratch and release
 * it: in stream order, and before returning).  The work split (and so the workspace
 * size) follows the compute-unit count of the current device: query with the
 * device current that the call will run on.  The library keeps no allocations
 * between calls, except the fixed scratch array of fgmm_iso_estep_f32_noalloc.
 * Calls are re-entrant given distinct outputs and workspaces.
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
    FGMM_ERR_UNSUPPORTED = -2, /* shape outside the supported range (e.g. full D > 4096) */
    FGMM_ERR_WORKSPACE = -3,   /* workspace smaller than *_workspace_bytes() */
    FGMM_ERR_HIP = -4,         /* a HIP runtime call or kernel launch failed */
    FGMM_ERR_SOURCE = -5,      /* a host row source returned an error */
    FGMM_ERR_SCRATCH = -6,     /* the call needs more than the no-allocation entry point's scratch */
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
    /* The accumulation pass skips every matrix-core step whose responsibilities
     * are all exactly zero, since such a step adds nothing, and the rows whose
     * responsibilities pass 1 proved zero for a component block.  DENSE runs
     * every step and every row (for timing the dense contraction).  With the
     * stored log-joint the results are bitwise the same either way; on the
     * default plan, whose pass 2 gathers the needed rows into tiles, the
     * statistics add the same nonzero terms in other groupings (last-bit
     * differences; logZ is the same). */
    FGMM_FLAG_DENSE = 1u << 5,
    /* The default plan: the workspace is O(N + K*D) (plus one need bit per
     * row and 32-component block) and pass 2 recomputes the D-contraction for
     * the (row, component block) pairs pass 1 marked as able to carry a nonzero
     * responsibility.  The N x K log-joint is never materialised.  Setting this
     * bit selects the default explicitly and overrides STORE_LOGJOINT. */
    FGMM_FLAG_RECOMPUTE = 1u << 6,
    /* The bf16 operand contract of the reference's H100 kernels, fp32 accumulation
     * and log-sum-exp throughout (the reference states a 5e-3 tolerance against
     * fp32 for it, flash_gmm_h100.py:276):
     *   isotropic (flash_gmm_h100.py:247-328): X and mu rounded to bfloat16 for x.mu
     *     and r^T X (r rounded there); constants from the fp32 mu.
     *   diagonal (flash_gmm_diag_h100.py:63-130, :159-282, :317-343): x, x^2,
     *     exp(-lss)/2 log2 e and mu exp(-lss)/2 log2 e rounded to bfloat16; r rounded
     *     for r^T x and r^T x^2.
     *   full (flash_gmm_full_h100.py:71-228, :289-298): x and L rounded to bfloat16
     *     for the whitening, L^T mu fp32; r rounded for mu_acc and r x_d2 for
     *     sig_outer[k][d2][:], which is then not exactly symmetric.  This path
     *     stores the log-joint, at most 16 GiB of it at a time: larger N runs as
     *     consecutive row chunks of 16 GiB / (4 K_padded) rows on one workspace
     *     (fgmm_full_workspace_bytes_ex sizes it for one chunk), each chunk adding
     *     its statistics to the outputs, so the sums round once per chunk.  A
     *     PHASE1 / PHASE2 call that needs more than one chunk returns
     *     FGMM_ERR_UNSUPPORTED.
     * FGMM_FLAG_RECOMPUTE and STORE_LOGJOINT have no effect with it. */
    FGMM_FLAG_BF16 = 1u << 7,
    /* Opt-in: pass 1 also stores the fp32 log-joint (N/32 x K/32 tiles of
     * 4 KiB, when that is at most 16 GiB, 32 < D <= 256 (full: D <= 128) and
     * K > 96) in the workspace,
     * and pass 2 reads it back instead of recomputing the D-contraction.  The
     * workspace is then O(N*K) (4.3 GB at N=1M, K=1024): size it with
     * *_workspace_bytes_ex(..., flags).  Calls that split the phases must agree
     * on this flag. */
    FGMM_FLAG_STORE_LOGJOINT = 1u << 9,
    /* Opt-in, isotropic model up to D = 128, diagonal up to D = 96, full up to
     * D = 64 and K = 512 (elsewhere it has no effect): the default plan plus a
     * stored-log-joint branch that the device selects per call.  A probe samples
     * up to 64 tiles of 32 rows before pass 1; when at least half of their (row,
     * component block) pairs (full: (row, component)) can carry a nonzero
     * responsibility (dense data, e.g. the reference's X, mu ~ N(0, I)
     * benchmark), pass 1 also stores the log-joint (iso, diag: with the rows'
     * split features and logZ pairs) and pass 2 reads them instead of recomputing
     * the contraction; otherwise the call runs as the default plan.  No host
     * synchronisation; the workspace is O(N*K) (about 4.7 GB at N=1M, K=1024,
     * D=128 isotropic, 5.4 GB at D=96 diagonal, 0.26 GB at N=250K, K=256
     * full: size it with *_workspace_bytes_ex) and the branch applies while the
     * log-joint fits in 16 GiB.  STORE_LOGJOINT and RECOMPUTE take precedence. */
    FGMM_FLAG_STORE_LOGJOINT_AUTO = 1u << 10,
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
/* log_sigma_sq and log_pi are contiguous (K).  Any D >= 1.  Above D = 256   */
/* the bf16 contract stores the N x K log-joint (16 GiB at most per call:     */
/* larger N runs as row chunks, as the full model's bf16 contract does).      */
/* ------------------------------------------------------------------------ */
size_t fgmm_iso_workspace_bytes(int64_t N, int64_t K, int64_t D);
/* Workspace for a call made with `flags` (FGMM_FLAG_STORE_LOGJOINT, RECOMPUTE
 * and BF16 matter); with flags = 0 it equals fgmm_iso_workspace_bytes(). */
size_t fgmm_iso_workspace_bytes_ex(int64_t N, int64_t K, int64_t D, unsigned flags);

int fgmm_iso_estep_f32(const float *X, int64_t ldx, int64_t N, int64_t D,
                       const float *mu, int64_t ldmu, int64_t K,
                       const float *log_sigma_sq, const float *log_pi,
                       float *logZ, float *Nk, float *mu_acc, float *sig_acc,
                       void *workspace, size_t workspace_bytes,
                       unsigned flags, void *stream);

/* ------------------------------------------------------------------------ */
/* Isotropic E-step that allocates nothing.  No counterpart in the reference:  */
/* for callers that cannot allocate device memory (code under HIP graph        */
/* capture, tight serving loops, harnesses that forbid hipMalloc).  The same   */
/* computation and results as fgmm_iso_estep_f32 with the same flags, with its */
/* workspace in a fixed device-resident scratch array of                       */
/* FGMM_NOALLOC_SCRATCH_BYTES per GPU.  The array is the only content of its   */
/* own code object, which HIP loads on a GPU at its first use there: the first */
/* noalloc call on that GPU reserves it (other entry points never do; with     */
/* deferred loading off, HIP_ENABLE_DEFERRED_LOADING=0, every code object is   */
/* loaded with the library), and it is held until the process ends.  A call   */
/* whose workspace (fgmm_iso_workspace_bytes_ex with the same flags) exceeds   */
/* it (above about 1.5M rows at K=1024, D=128) runs as consecutive row chunks  */
/* on the array, each after the first adding its statistics to the outputs:   */
/* logZ is the one-call result per row, the statistics round once per chunk.   */
/* Such a call with FGMM_FLAG_PHASE1 or PHASE2, or one where not even 256 rows */
/* fit, returns FGMM_ERR_SCRATCH.                                              */
/* FGMM_FLAG_STORE_LOGJOINT is rejected (FGMM_ERR_INVALID_ARG).  Every call on */
/* a GPU uses that GPU's one array: calls that overlap on one GPU (different   */
/* streams or host threads without ordering) race, and a PHASE2 call reads     */
/* what the last PHASE1 call on that GPU left.                                 */
/* ------------------------------------------------------------------------ */
#define FGMM_NOALLOC_SCRATCH_BYTES ((size_t)64 << 20)

int fgmm_iso_estep_f32_noalloc(const float *X, int64_t ldx, int64_t N, int64_t D,
                               const float *mu, int64_t ldmu, int64_t K,
                               const float *log_sigma_sq, const float *log_pi,
                               float *logZ, float *Nk, float *mu_acc, float *sig_acc,
                               unsigned flags, void *stream);

/* ------------------------------------------------------------------------ */
/* Diagonal-covariance E-step.                                               */
/* Replaces flash_gmm_estep_diag(X, mu, log_sigma_sq, log_pi) at             */
/* flash_gmm_diag_h100.py:305-384.  log_sigma_sq is K x D with row stride     */
/* ldlss; sig_acc is K x D:                                                   */
/*   ll_nk      = log_pi_k - 0.5*(D log(2 pi) + sum_d lss_kd)                 */
/*                - 0.5 * sum_d (x_nd - mu_kd)^2 exp(-lss_kd)                 */
/*   sig_acc_kd = sum_n r_nk (x_nd - mu_kd)^2                                 */
/* Any D >= 1 (above D = 256 the bf16 contract stores the log-joint, as the  */
/* isotropic one does).                                                       */
/* ------------------------------------------------------------------------ */
size_t fgmm_diag_workspace_bytes(int64_t N, int64_t K, int64_t D);
size_t fgmm_diag_workspace_bytes_ex(int64_t N, int64_t K, int64_t D, unsigned flags);

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
/* Supports 1 <= D <= 4096 (the bf16 contract and the stored log-joint:       */
/* D <= 128) and K * u(u+1)/2 < 2^24 with u = ceil(D / 32).  Above D = 256    */
/* pass 1 always stores the N x K log-joint (pass 2 reads r from it); calls   */
/* whose log-joint would exceed 16 GiB run as row chunks, as with the bf16    */
/* contract (a PHASE1 / PHASE2 call that needs more than one chunk returns    */
/* FGMM_ERR_UNSUPPORTED).                                                     */
/* ------------------------------------------------------------------------ */
size_t fgmm_full_workspace_bytes(int64_t N, int64_t K, int64_t D);
size_t fgmm_full_workspace_bytes_ex(int64_t N, int64_t K, int64_t D, unsigned flags);

int fgmm_full_estep_f32(const float *X, int64_t ldx, int64_t N, int64_t D,
                        const float *mu, int64_t ldmu, int64_t K,
                        const float *prec_chol, const float *log_pi,
                        float *logZ, float *Nk, float *mu_acc, float *sig_outer,
                        void *workspace, size_t workspace_bytes,
                        unsigned flags, void *stream);

/* ------------------------------------------------------------------------ */
/* Host row sources for the streaming driver.                                */
/* A row source fills dst (host memory, nrows x D floats, row stride D) with  */
/* rows [row0, row0 + nrows) of the data set and returns 0, or a nonzero     */
/* status that aborts the stream.  It replaces the README's `for chunk in     */
/* dataloader: chunk.cuda()` recipe (README.md:86-96).                        */
/* ------------------------------------------------------------------------ */
typedef int (*fgmm_row_source_fn)(void *user, int64_t row0, int64_t nrows, int64_t D, float *dst);

/* Built-in synthetic source: x_n = centres[a_n] + z_n with a_n uniform over K
 * and z_n ~ N(0, I), counter-based (Philox4x32-10 keyed by seed, counter = row
 * index), so a row's value does not depend on how the rows are chunked.  No
 * counterpart in the reference (its benchmark draws torch.randn on the GPU,
 * flash_gmm.py:231). */
typedef struct fgmm_synth_iso {
    const float *centres; /* host, K x D, row-major */
    int64_t K, D;
    uint64_t seed;
    int threads;          /* host threads; 0 = all hardware threads */
} fgmm_synth_iso;

int fgmm_synth_iso_source(void *user, int64_t row0, int64_t nrows, int64_t D, float *dst);

/* Row sources over local vector files, the layouts the reference's tuning    */
/* data sets are distributed in (SIFT1M, GIST1M: .fvecs; SIFT1B: .bvecs;       */
/* Deep1B / Deep10M: .fbin, .u8bin; flash_gmm_diag_h100.py:17,299-301 names    */
/* SIFT1M, GloVe and Deep10M, and the reference ships no reader).  The file is */
/* memory-mapped; N and D come from its headers; byte values become floats.    */
/* fgmm_vecs_open returns FGMM_ERR_SOURCE when the file cannot be opened or    */
/* mapped and FGMM_ERR_INVALID_ARG for a malformed header.  Pass the           */
/* fgmm_vecs_file as the `user` of fgmm_vecs_source.                           */
/* ------------------------------------------------------------------------ */
enum fgmm_vecs_format {
    FGMM_VECS_FVECS = 0,   /* per vector: int32 d, then d float32 */
    FGMM_VECS_BVECS = 1,   /* per vector: int32 d, then d uint8 */
    FGMM_VECS_FBIN = 2,    /* uint32 n, uint32 d, then n*d float32 */
    FGMM_VECS_U8BIN = 3,   /* uint32 n, uint32 d, then n*d uint8 */
};

typedef struct fgmm_vecs_file {
    void *base;            /* mapping (owned; release with fgmm_vecs_close) */
    size_t bytes;
    int64_t N, D;          /* vectors and dimensions in the file */
    int format;            /* fgmm_vecs_format */
    int threads;           /* host threads per chunk; 0 = all hardware threads */
} fgmm_vecs_file;

int fgmm_vecs_open(const char *path, int format, int threads, fgmm_vecs_file *f);
int fgmm_vecs_source(void *user, int64_t row0, int64_t nrows, int64_t D, float *dst);
void fgmm_vecs_close(fgmm_vecs_file *f);

/* ------------------------------------------------------------------------ */
/* Isotropic M-step on the device (README.md:59-61):                          */
/*   log_pi = log(Nk / N),  mu = mu_acc / Nk,                                 */
/*   sigma^2 = max(var_floor, sig_acc / (D Nk) [- ||mu_new - mu_old||^2 / D]) */
/* The bracketed term is applied with FGMM_MSTEP_EXACT_VARIANCE (sig_acc is    */
/* accumulated about the old means).  Components with Nk = 0 keep mu and      */
/* log_sigma_sq and get log_pi = -inf.  mu (K x D, row stride ldmu),           */
/* log_sigma_sq and log_pi (K) are updated in place.                          */
/* ------------------------------------------------------------------------ */
enum { FGMM_MSTEP_EXACT_VARIANCE = 1u << 8 };

int fgmm_iso_mstep_f32(const float *Nk, const float *mu_acc, const float *sig_acc,
                       int64_t N, int64_t K, int64_t D, double var_floor,
                       float *mu, int64_t ldmu, float *log_sigma_sq, float *log_pi,
                       unsigned flags, void *stream);

/* ------------------------------------------------------------------------ */
/* Diagonal-covariance M-step on the device (the per-dimension analogue of    */
/* README.md:59-61): log_pi = log(Nk/N), mu = mu_acc/Nk,                       */
/* sigma^2_kd = max(var_floor, sig_acc_kd/Nk [- (mu_new - mu_old)_d^2]), the   */
/* bracket applied with FGMM_MSTEP_EXACT_VARIANCE.  mu (K x D, stride ldmu),    */
/* log_sigma_sq (K x D, stride ldlss) and log_pi are updated in place;        */
/* components with Nk = 0 keep mu and log_sigma_sq and get log_pi = -inf.     */
/* ------------------------------------------------------------------------ */
int fgmm_diag_mstep_f32(const float *Nk, const float *mu_acc, const float *sig_acc,
                        int64_t N, int64_t K, int64_t D, double var_floor,
                        float *mu, int64_t ldmu, float *log_sigma_sq, int64_t ldlss,
                        float *log_pi, unsigned flags, void *stream);

/* ------------------------------------------------------------------------ */
/* Full-covariance M-step on the device, producing the E-step's own input     */
/* parameterisation (flash_gmm_full_h100.py:238,257-260):                      */
/*   Sigma_k = sig_outer_k / Nk_k - mu_k mu_k^T + reg_covar I                 */
/*   prec_chol_k = L_k lower-triangular, L_k L_k^T = Sigma_k^-1, positive diag */
/* computed in fp64 per component.  mu (K x D, stride ldmu), prec_chol         */
/* (K x D x D contiguous) and log_pi are written; components with Nk = 0 keep  */
/* mu and prec_chol and get log_pi = -inf.  info (device int, may be NULL,     */
/* zeroed by the caller) is incremented for every component whose Sigma was  */
/* not positive definite (its failing pivots are replaced by reg_covar).      */
/* Supports 1 <= D <= 4096.  Above D = 128 the fp64 matrices of each component */
/* live in device scratch the call allocates and frees in stream order         */
/* (hipMallocAsync / hipFreeAsync, at most 1 GiB; components run in batches);  */
/* the work is O(D^3) per component.                                          */
/* ------------------------------------------------------------------------ */
int fgmm_full_mstep_f32(const float *Nk, const float *mu_acc, const float *sig_outer,
                        int64_t N, int64_t K, int64_t D, double reg_covar,
                        float *mu, int64_t ldmu, float *prec_chol, float *log_pi,
                        int *info, void *stream);

/* ------------------------------------------------------------------------ */
/* Streaming isotropic EM for data sets larger than device memory.           */
/* Replaces the README recipe at README.md:81-103 (pageable chunk.cuda() per  */
/* chunk, accumulators summed in Python, M-step in PyTorch).  Rows come from   */
/* `src` into two pinned host buffers of chunk_rows rows; host filling, the   */
/* host-to-device copy (copy stream) and the E-step (compute stream) of       */
/* consecutive chunks overlap, also across iterations (the rows do not       */
/* depend on the parameters).  After every pass over the N rows (N >= 1) the  */
/* M-step updates mu (K x D contiguous), log_sigma_sq and log_pi in place     */
/* (device pointers).  The call allocates its buffers and frees them before   */
/* it returns; it blocks until the last iteration is done.                    */
/* ------------------------------------------------------------------------ */
#define FGMM_EM_MAX_REPORTED_ITERS 16

typedef struct fgmm_em_config {
    int64_t N, K, D;         /* rows, components, dimensions (any D >= 1) */
    int64_t chunk_rows;      /* rows per host chunk */
    int iterations;          /* EM iterations */
    double var_floor;        /* lower bound on sigma^2 in the M-step */
    unsigned mstep_flags;    /* FGMM_MSTEP_* */
} fgmm_em_config;

typedef struct fgmm_em_report {
    int iterations;
    double total_ms;         /* wall time of the call */
    double source_ms;        /* host time spent in the row source */
    double h2d_ms;           /* device time of the host-to-device copies */
    double estep_ms;         /* device time of the E-steps (incl. logZ sums) */
    double mstep_ms;         /* device time of the M-steps */
    size_t device_bytes;     /* device memory allocated by the call (peak) */
    size_t pinned_bytes;     /* pinned host memory allocated by the call */
    double loglik[FGMM_EM_MAX_REPORTED_ITERS]; /* sum_n logZ_n per iteration, before its M-step */
    double setup_ms;         /* wall time spent allocating streams, events and buffers */
} fgmm_em_report;

int fgmm_stream_em_iso(const fgmm_em_config *cfg, fgmm_row_source_fn src, void *user,
                       float *mu, float *log_sigma_sq, float *log_pi, fgmm_em_report *report);

#ifdef __cplusplus
}
#endif

#endif /* FLASHGMM_H */
