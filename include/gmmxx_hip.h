/*
 * gmmxx_hip.h — C ABI of the MI355X (gfx950) GMM EM engine.
 *
 * The library replaces the reference's native extension `gmmxx._C`
 * (gmmxx/csrc/bindings.cpp:16-191, loaded by gmmxx/_cuda.py:25-32) and the
 * Triton E/M-step modules for the EM iteration hot path.  All entry points:
 *   - take plain device pointers, sizes and a hipStream_t passed as void*;
 *   - allocate nothing: scratch memory comes from the caller's workspace
 *     (size from gmmxx_hip_workspace_bytes), outputs are caller-owned;
 *   - are asynchronous on the given stream and never synchronise;
 *   - return GMMXX_OK (0) or a nonzero status; the message for the calling
 *     thread is available from gmmxx_hip_last_error().
 * Data layout: x is row-major (B, N, D) fp32 or bf16; every parameter array is
 * fp32 row-major in the reference's batched shapes: means (B, K, D), weights
 * (B, K), covariances spherical (B, K), diag (B, K, D), tied (B, D, D),
 * full (B, K, D, D).  With bf16 x (spherical) the means are bf16 values, as the
 * reference keeps them in x's dtype (gmmxx/torch_fallback.py:2295): every call
 * computes with the means rounded to bf16, and the M-step stores them rounded
 * (the variance is formed from the unrounded mean).
 */
#ifndef GMMXX_HIP_H_
#define GMMXX_HIP_H_

#include <stdint.h>

#ifdef __cplusplus
extern "C" {
#endif

#define GMMXX_HIP_ABI_VERSION 2

enum gmmxx_status {
  GMMXX_OK = 0,
  GMMXX_ERR_INVALID_ARGUMENT = 1,
  GMMXX_ERR_UNSUPPORTED = 2,
  GMMXX_ERR_WORKSPACE = 3,
  GMMXX_ERR_HIP = 4
};

enum gmmxx_covariance { GMMXX_SPHERICAL = 0, GMMXX_DIAG = 1, GMMXX_TIED = 2, GMMXX_FULL = 3 };
enum gmmxx_dtype { GMMXX_F32 = 0, GMMXX_BF16 = 1, GMMXX_F16 = 2 };

/* param_dtype: the dtype the parameters are kept in between iterations.  The
 * finalize rounds the new means, and for diag/tied/full also the covariances
 * and weights, to it (stored in the fp32 buffers), as the reference's M-step
 * casts them to x's dtype (gmmxx/torch_fallback.py:2295, :2654-2666,
 * :3143-3167) when a half-precision x is computed in fp32.  GMMXX_F32 (0, a
 * zero-initialised descriptor) keeps them unrounded; bf16 x (spherical) implies
 * bf16 means.  `reserved` must be 0. */
typedef struct gmmxx_problem {
  int32_t covariance_type; /* enum gmmxx_covariance */
  int32_t x_dtype;         /* enum gmmxx_dtype: GMMXX_F32 or GMMXX_BF16 */
  int64_t B, N, D, K;
  int32_t param_dtype;     /* enum gmmxx_dtype */
  int32_t reserved;
} gmmxx_problem;

/* ABI version of the loaded library (GMMXX_HIP_ABI_VERSION). */
int gmmxx_hip_abi_version(void);

/* Thread-local message of the last failing call on this thread ("" if none). */
const char* gmmxx_hip_last_error(void);

/* Smoke test: out[i] = in[i] + offset.
 * Replaces `canary_add_offset` (gmmxx/csrc/canary/canary.cu:21-48, gmmxx/_cuda.py:67-95). */
int gmmxx_hip_canary(const int32_t* in, int32_t* out, int64_t n, int32_t offset, void* stream);

/* Properties of device `device` as the engine sees them.  `supported` is 1 for
 * gfx950 (the only target the library is built for); `coop_capacity` is the
 * number of co-resident workgroups of the single-pass cooperative kernel.
 * Replaces the device checks of the reference's runtime gates and
 * require_cuda / has_cuda (gmmxx/_runtime.py:31-191, gmmxx/_cuda.py:44-64),
 * which probe torch.cuda.get_device_capability. */
typedef struct gmmxx_dev_info {
  int32_t device;
  int32_t supported;          /* 1: gfx950 */
  char arch[64];              /* e.g. "gfx950:sramecc+:xnack-" */
  int32_t compute_units;
  int32_t wave_size;
  int32_t clock_khz;
  int32_t coop_capacity;
  int64_t hbm_bytes;
  int64_t lds_per_workgroup;
} gmmxx_dev_info;
int gmmxx_hip_device_info(int device, gmmxx_dev_info* out);

/* 1 if the engine supports the problem shape/dtype, else 0: D <= 128 for every
 * covariance type, K <= 65536, B <= 65535, x fp32 (or bf16 for spherical).
 * Replaces the shape gates cuda_{spherical,diag,tied,full}_supported
 * (gmmxx/_runtime.py:31-191). */
int gmmxx_hip_supported(const gmmxx_problem* p);

/* Bytes of device workspace every entry point below needs for this problem
 * (the same size serves all of them); -1 if unsupported. */
int64_t gmmxx_hip_workspace_bytes(const gmmxx_problem* p);

/* One full soft-EM iteration, in place: the iteration prelude (variance clamp
 * to reg_covar for spherical/diag, weight floor min_weight and
 * renormalisation), the E-step log-normaliser and responsibilities, the M-step
 * sufficient statistics and the finalize.  `lower_bound` (device, 1 float)
 * receives the mean per-sample log-likelihood under the parameters on entry.
 * `gram` is XᵀX per batch (B, D, D) for tied (gmmxx_hip_gram), NULL otherwise.
 * Replaces one loop iteration of batch_gmm_{Spherical,Diagonal}_torch_native
 * and _batch_gmm_matrix_torch_native (gmmxx/torch_fallback.py:2060-2330,
 * :2484-2698, :2864-3199) and the CUDA loops _train_{spherical,diag,tied,full}_cuda
 * (gmmxx/interface.py:666-1275) with their _C calls spherical_fused,
 * blocked_update_*, finalize_* (gmmxx/csrc/bindings.cpp:60-170). */
int gmmxx_hip_em_step(const gmmxx_problem* p, const void* x, float* means, float* covariances,
                      float* weights, const float* gram, double reg_covar, double min_weight,
                      float* lower_bound, void* workspace, int64_t workspace_bytes, void* stream);

/* Asynchronous failures of earlier calls on this workspace: the word is nonzero
 * when a single pass whose workgroups exchange row partials gave up waiting for
 * a partner workgroup (the members of a group were not all resident: another
 * kernel or process held part of the GPU).  Two passes do this: the cooperative
 * kernel (spherical bf16 at D = 128, 256 < K <= 1024; GMMXX_HIP_NO_COOP=1
 * selects two passes instead) and the exchange pass (fp32 x: spherical at
 * D <= 128, tied and diag at D <= 64, each with 256 < K <= 1024, i.e. two to
 * four component tiles of 256; GMMXX_HIP_NO_XCH=1 selects two passes
 * instead).  Such an iteration writes NaN to its lower bound (or ll_sum) and
 * leaves the parameters unchanged.  A non-finite input row does not stall the
 * exchange: it propagates into the lower bound and parameters as in the
 * reference, and the word stays 0.  Copies the word into *status_out (device
 * memory, 1 uint32) and clears it, stream-ordered.  A newly allocated workspace holds arbitrary
 * bytes: zero it, or call this once and discard the result, before the calls
 * whose status is wanted.  No reference counterpart: the reference's kernels
 * report errors synchronously through TORCH_CHECK (gmmxx/_cuda.py:41-54); this
 * is how the asynchronous C ABI reports its one asynchronous failure. */
int gmmxx_hip_take_status(const gmmxx_problem* p, void* workspace, int64_t workspace_bytes,
                          uint32_t* status_out, void* stream);

/* gmmxx_hip_em_step without a caller workspace: the same kernels run on a
 * static device scratch array of the library (64 MiB per device, held for
 * the life of the process), so the call allocates nothing and takes no
 * workspace arguments.  Problems whose gmmxx_hip_workspace_bytes exceeds
 * 64 MiB are refused with GMMXX_ERR_WORKSPACE before any launch.  Every call
 * on one device shares that device's scratch: calls that overlap on one
 * device (two streams, two threads) race and must be ordered by the caller.
 * The call clears the scratch's status words first and there is no workspace
 * to pass to gmmxx_hip_take_status, so a single pass that timed out waiting
 * for a partner workgroup (see gmmxx_hip_take_status) shows only as a NaN
 * *lower_bound with the parameters left unchanged: check the lower bound.
 * Call with the stream's device current.  No counterpart in the reference:
 * it is for callers that cannot allocate device memory (code under HIP graph
 * capture, tight serving loops, harnesses that forbid hipMalloc). */
int gmmxx_hip_em_step_noalloc(const gmmxx_problem* p, const void* x, float* means, float* covariances,
                              float* weights, const float* gram, double reg_covar, double min_weight,
                              float* lower_bound, void* stream);

/* The six phases of gmmxx_hip_em_step, for callers that time or interleave
 * them; gmmxx_hip_em_step(...) == phases PREPARE..FINALIZE in order with the
 * same arguments and workspace.  PREPARE: iteration prelude, Cholesky
 * (tied/full), E-step operand packing, tied row forms.  LSE_TILE: the
 * log-normaliser tile kernel.  COMBINE: per-row merge of the component tiles
 * and the lower bound.  STATS_TILE: the responsibilities x statistics tile
 * kernel.  REDUCE: ordered sum of the per-slice statistics.  FINALIZE: M-step
 * parameter update.  Same role as the reference's separate _C ops
 * prepare_spherical_estep / spherical_logsumexp / blocked_update_* /
 * finalize_* (gmmxx/csrc/bindings.cpp:28-170). */
enum gmmxx_em_phase {
  GMMXX_PHASE_PREPARE = 0,
  GMMXX_PHASE_LSE_TILE = 1,
  GMMXX_PHASE_COMBINE = 2,
  GMMXX_PHASE_STATS_TILE = 3,
  GMMXX_PHASE_REDUCE = 4,
  GMMXX_PHASE_FINALIZE = 5
};
int gmmxx_hip_em_phase(const gmmxx_problem* p, int phase, const void* x, float* means,
                       float* covariances, float* weights, const float* gram, double reg_covar,
                       double min_weight, float* lower_bound, void* workspace,
                       int64_t workspace_bytes, void* stream);

/* E-step + M-step sufficient statistics only (no finalize, parameters untouched;
 * the iteration prelude is applied to the values used).  Outputs (device):
 *   nk (B, K); sum_x (B, K, D); sum_q: spherical Σ r‖x‖² (B, K), diag Σ r x² (B, K, D),
 *   full Σ r xxᵀ (B, K, D, D), tied: pass NULL; ll_sum (1 float): Σ over all rows of
 *   log Σ_k w_k N(x | k).
 * Replaces the statistics kernels blocked_update_* / spherical_fused / the
 * Triton fused_single_tile_update_* (gmmxx/csrc/bindings.cpp:104-170,
 * gmmxx/fused_update_triton.py:449-659). */
int gmmxx_hip_estep_stats(const gmmxx_problem* p, const void* x, const float* means,
                          const float* covariances, const float* weights, double reg_covar,
                          double min_weight, float* nk, float* sum_x, float* sum_q, float* ll_sum,
                          void* workspace, int64_t workspace_bytes, void* stream);

/* Approximate top-k E-step statistics: like gmmxx_hip_estep_stats, but each
 * row's responsibilities cover only its top_k components (largest logits,
 * ties to the lower component index), normalised over those, and ll_sum sums
 * the top-k log-normalisers.  1 <= top_k <= K-1 (top_k >= K is exact EM: use
 * gmmxx_hip_estep_stats).  For top_k > 1 the (B, N, K) logits are materialised
 * in the workspace, whose size is gmmxx_hip_topk_workspace_bytes(p, top_k);
 * callers bound it by passing row chunks, as the reference does with
 * chunk_size_N.  top_k = 1 (hard assignment to the first maximum) stores no
 * logits and needs only O(B·N) beyond the plan's workspace.
 * Replaces _topk_logits_for_chunk + _accumulate_topk_stats
 * (gmmxx/torch_fallback.py:667-777, used by the EM loops at :2101-2145,
 * :2504-2526, :2915-2936) and the CUDA/Triton approximate updates
 * (gmmxx/_cuda.py:783-889, gmmxx/approx_update_triton.py:25-281). */
int64_t gmmxx_hip_topk_workspace_bytes(const gmmxx_problem* p, int top_k);
int gmmxx_hip_estep_stats_topk(const gmmxx_problem* p, const void* x, const float* means,
                               const float* covariances, const float* weights, double reg_covar,
                               double min_weight, int top_k, float* nk, float* sum_x, float* sum_q,
                               float* ll_sum, void* workspace, int64_t workspace_bytes, void* stream);

/* M-step finalize from sufficient statistics, in place on (means, covariances,
 * weights): nk (B, K), sum_x (B, K, D) and sum_q as gmmxx_hip_estep_stats returns
 * them (spherical Σ r‖x‖² (B, K), diag Σ r x² (B, K, D), full Σ r xxᵀ (B, K, D, D),
 * tied NULL and gram = XᵀX (B, D, D) instead), summed over any number of row
 * chunks; p->N is the total row count per batch (the weights' denominator).
 * Components with N_k <= min_weight keep their mean and (clamped) covariance.
 * The workspace needs gmmxx_hip_workspace_bytes of p with N = 1 (any larger N
 * also serves).  Used by the large-N streaming fit, which accumulates the chunk
 * statistics itself.  Replaces the finalize ops finalize_spherical(_soft) /
 * finalize_diag (gmmxx/csrc/bindings.cpp:124-146, :170; gmmxx/_cuda.py:758,
 * :1029), tied_finalize / full_finalize (gmmxx/_cuda.py:1204-1238, :1355-1416)
 * and the finalize block of the large-N loop (gmmxx/large_n.py:1496-1537). */
int gmmxx_hip_finalize_stats(const gmmxx_problem* p, const float* nk, const float* sum_x, const float* sum_q,
                             const float* gram, double reg_covar, double min_weight, float* means,
                             float* covariances, float* weights, void* workspace, int64_t workspace_bytes,
                             void* stream);

/* Inference under fixed parameters (no prelude): per-sample log-likelihood
 * `scores` (B, N) and/or first-maximum labels (B, N) int64; either may be NULL.
 * Replaces spherical/diag/full assign + logsumexp (gmmxx/csrc/bindings.cpp:19-58,
 * :140-190; gmmxx/_cuda.py:1246-1314) and the torch inference functions
 * *_assign_torch_native_chunked / *_score_samples_torch_native_chunked
 * (gmmxx/torch_fallback.py:780-1130). */
int gmmxx_hip_score(const gmmxx_problem* p, const void* x, const float* means,
                    const float* covariances, const float* weights, float* scores, int64_t* labels,
                    void* workspace, int64_t workspace_bytes, void* stream);

/* Responsibilities (B, N, K) fp32 under fixed parameters.
 * Replaces *_resp (gmmxx/csrc/bindings.cpp:40-58) and
 * *_predict_proba_torch_native_chunked (gmmxx/torch_fallback.py:1133-1345). */
int gmmxx_hip_predict_proba(const gmmxx_problem* p, const void* x, const float* means,
                            const float* covariances, const float* weights, float* proba,
                            void* workspace, int64_t workspace_bytes, void* stream);

/* predict_proba and score_samples from one E-step: responsibilities (B, N, K)
 * and per-sample log-likelihood (B, N), either may be NULL (not both).  When
 * every component fits one tile workgroup the single responsibility pass forms
 * the row log-normalisers itself and writes them as the scores; otherwise the
 * log-normaliser pass writes the scores and the responsibility pass reuses its
 * log-normalisers.  Replaces the estimator's predict_proba + score_samples pair
 * (gmmxx/interface.py:2138-2203, :2412-2467), each of which runs its own
 * streamed log-normaliser (gmmxx/torch_fallback.py:1279-1345, :1094-1130); one
 * entry for every covariance type, the full-covariance pair included. */
int gmmxx_hip_predict_proba_score(const gmmxx_problem* p, const void* x, const float* means,
                                  const float* covariances, const float* weights, float* proba,
                                  float* scores, void* workspace, int64_t workspace_bytes, void* stream);

/* XᵀX per batch (B, D, D) fp32, the fit-constant of the tied M-step
 * (gmmxx/torch_fallback.py:2856-2862). */
int gmmxx_hip_gram(const gmmxx_problem* p, const void* x, float* out, void* workspace,
                   int64_t workspace_bytes, void* stream);

/* Greedy k-means++ seeding of K centres (B, K, D) fp32 from a row sample
 * (B, S, D) fp32: centre 0 is row first_idx[b] (int64, clamped to [0, S)); each
 * later centre c is the best of `trials` candidates drawn by D² sampling with
 * the uniform numbers draws[b][c-1][0..trials) in [0, 1) -- the row where the
 * running sum of squared distances to the nearest centre first reaches
 * u·total (the last row beyond the total, row 0 when the total is 0) -- best
 * meaning the least potential Σ_i min(closest_i, ‖s_i - c‖²), first on ties.
 * 1 <= K <= S <= 65536, D <= 1024, trials <= 16.  The workspace takes
 * gmmxx_hip_kmeans_pp_workspace_bytes bytes (-1: arguments out of range).
 * Replaces _kmeans_plus_plus_init_means (gmmxx/torch_fallback.py:1390-1451),
 * which draws the same numbers with torch.randint / torch.rand. */
int64_t gmmxx_hip_kmeans_pp_workspace_bytes(int64_t B, int64_t S, int64_t D, int64_t K, int trials);
int gmmxx_hip_kmeans_pp(const float* sample, int64_t B, int64_t S, int64_t D, int64_t K, int trials,
                        const int64_t* first_idx, const float* draws, float* centers, void* workspace,
                        int64_t workspace_bytes, void* stream);

#ifdef __cplusplus
}
#endif

#endif /* GMMXX_HIP_H_ */
