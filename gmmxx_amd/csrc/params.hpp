// Component-side kernels: argument blocks and host launchers.
#pragma once

#include <hip/hip_runtime.h>
#include <stdint.h>

namespace gx {

struct PrepArgs {
  int cov, bf, prelude;
  int param_round;         // 1 bf16, 2 fp16: the prelude's normalised weights kept in that dtype
  int B, K, D, DP, EP;
  float reg_covar, min_weight;
  const float* means;      // [B][K][D]
  const float* covs;       // spherical [B][K], diag [B][K][D]
  const float* weights;    // [B][K]
  const float* prec;       // tied [B][D][D], full [B][K][D][D]
  const int* first_ok;     // full: per-matrix first jitter level of the Cholesky ladder
  const int* chol_level;   // full: the batch's jitter level (written by launch_chol's kernels)
  const float* logdet;     // tied [B], full [B][K]
  float* covs_used;        // spherical/diag: the (clamped) variances this iteration used
  void* w_hi;              // [B][K][EP]
  void* w_lo;              // [B][K][EP] (bf16 path)
  void* w_aug;             // [B][K][32] (spherical bf16 path)
  void* w_mu;              // [B][K][DP] spherical bf16 cooperative and fused passes: the bf16 means (or null)
  float* w_scale;          // [B][K] with w_mu: log2(e)/σ², the factor of the product x·μ
  void* w_augs;            // [B][K][16] fused pass: the augmented constants divided by that factor (or null)
  float4* cconst;          // [B][K]
  const float* gram;       // tied EM: XᵀX [B][D][D] (or null)
  double* shift;           // with gram: [B][D] row terms -½ Σ_j P_rj (XᵀX)_rj
};

struct CombineArgs {
  int B, ktiles;
  int64_t N;
  const float* part_ms;
  const int* part_idx;
  float* lse2;             // [B][N] or null
  float* scores;           // [B][N] natural-log scores or null
  int64_t* labels;         // [B][N] or null
  double* ll_part;         // [B][gridDim.x] or null
  int* idx32;              // [B][N] first argmax as int, or null (needs the argmax partials)
  int max_only;            // lse2 (and the log-likelihood) from the row maximum alone
};

struct FinalizeArgs {
  int cov, B, K, D, DP, JP, nk_col;
  int sq_col, sq_n;        // spherical: Σ r‖x‖² = Σ_{i < sq_n} stats[sq_col + i]
  int64_t N;
  float reg_covar, min_weight;
  const float* stats;      // [B][K][JP]
  const float* covs_used;  // spherical/diag old (clamped) variances
  const float* gram;       // tied XᵀX [B][D][D]
  float* means;
  float* covs;
  float* weights;
  const unsigned* skip;    // nonzero *skip: leave the parameters unchanged (or null)
  int bf_means;            // spherical bf16 x: store the means rounded to bf16
  int param_round;         // 1 bf16, 2 fp16: store the means (and, diag/tied/full, the
                           // covariances and weights) rounded to that dtype
};

struct UnpackArgs {
  int cov, K, D, DP, JP, nk_col;
  int sq_col, sq_n;
  const float* stats;
  float* nk;
  float* sum_x;
  float* sum_q;
};

// Inverse of UnpackArgs: caller-side statistics (N_k, Σ r x, Σ r q(x)) packed into
// the statistics rows, plus the variances an inactive component keeps
// (spherical/diag: max(covariance, reg_covar), the iteration prelude's clamp).
struct PackArgs {
  int cov, K, D, DP, JP, nk_col;
  int sq_col;
  float reg_covar;
  const float* nk;
  const float* sum_x;
  const float* sum_q;
  const float* covs;
  float* stats;
  float* covs_used;
};

void launch_prep(const PrepArgs& a, hipStream_t s);
// Padded order of the per-matrix factor buffer (lbuf: M x chol_dp(D)^2 floats).
int chol_dp(int D);
// first_ok: M per-matrix first levels, then the batch level (written by every path).
// linv (optional, M x D x D): X = L^-1 of the factor at the batch level, zeros
// above the diagonal; prec may then be null (X alone).
void launch_chol(const float* cov, int D, int M, int* first_ok, int* level, float* lbuf, float* prec,
                 float* logdet, hipStream_t s, float* linv = nullptr);
void launch_rowquad(const float* x, int B, int64_t N, int D, const float* prec, float* rowq, hipStream_t s);
int launch_combine(const CombineArgs& a, hipStream_t s);  // returns the per-batch block count
int combine_blocks(int64_t N);
void launch_ll_reduce(const double* ll_part, int count, double inv_total, float* out, hipStream_t s);
// out = Σ over slices of part[slice][M], in a fixed order; tmp (optional, tmp_floats
// long) lets many slices be summed in parallel groups first.
// A log-likelihood reduction folded into the last slice-reduction launch (one
// more workgroup): *out = Σ part[0 .. count) · inv_total; with status set
// (cooperative / exchange passes) a nonzero *status turns *out into NaN and is
// added to *sticky.
struct LlFold {
  const double* part;
  int count;
  double inv_total;
  float* out;
  const unsigned* status;
  unsigned* sticky;
};
void launch_reduce_slices(const float* part, int slices, int64_t M, float* out, hipStream_t s,
                          float* tmp = nullptr, int64_t tmp_floats = 0, const LlFold* ll = nullptr);
void launch_finalize(const FinalizeArgs& a, hipStream_t s);
void launch_unpack(const UnpackArgs& a, int B, hipStream_t s);
void launch_pack(const PackArgs& a, int B, hipStream_t s);
void launch_gram(const float* x, int B, int64_t N, int D, int slices, int64_t rows_per_slice, float* part,
                 hipStream_t s);
// p[0..n) = 0 (a kernel, not a memset: safe inside captured graphs).
void launch_zero_words(unsigned* p, int n, hipStream_t s);
// *out = *sticky; *sticky = 0.
void launch_take_status(unsigned* sticky, uint32_t* out, hipStream_t s);
void launch_canary(const int32_t* in, int32_t* out, int64_t n, int32_t offset, hipStream_t s);

}  // namespace gx
