// Internal launch interface between the C-ABI layer and the kernels.
#pragma once

#include <hip/hip_runtime.h>
#include <stdint.h>

namespace gx {

struct TileArgs {
  const void* x;               // [B][N][D], fp32 or bf16
  int vec_ok;                  // x rows are 16-byte aligned and D == DP
  int64_t N;
  int D, K, B;
  int ktiles;                  // component tiles per batch
  int64_t rows_per_slice;      // multiple of 32
  const void* w_hi;            // [B][K][EP] E-step operand (bf16 hi or fp32)
  const void* w_lo;            // [B][K][EP] bf16 lo part (bf16 path only)
  const void* w_aug;           // [B][K][32] bf16 augmented constants (spherical bf16 path)
  const void* w_mu;            // [B][K][DP] bf16 means (fused kernel)
  const float* w_scale;        // [B][K] log2(e)/σ², the factor of x·μ (fused kernel)
  const void* w_augs;          // [B][K][16] bf16 [-½ -½ -½ 0 0 0 C'_h C'_m | C'_l 0 ...] (fused kernel)
  const float4* cconst;        // [B][K] (A, C, 0, 0): l2 = A*(rowq - 2S) + C (spherical, tied) or A*S + C
  const float* rowq;           // [B][N] tied: xᵀPx
  const float* lse2;           // [B][N] log2-domain log-normaliser (STATS / PROBA)
  uint4* rowaux;               // [B][N] spherical bf16: augmented row chunk (written by LSE)
  float* part_ms;              // [ktiles][B][N][2] (max, scaled sum)   (LSE)
  int* part_idx;               // [ktiles][B][N] first argmax           (LSE)
  float* part_stats;           // [slices][B][K][JP]                    (STATS)
  float* proba;                // [B][N][K]                             (PROBA)
  float* scores;               // [B][N] natural-log row log-normalisers (PROBA_LSE, or null)
  int nslices;                 // row slices of the fused kernel
  double* ll_part;             // [B][nslices] partial log-likelihood   (fused)
  int raw_logits;              // PROBA: write the log2-domain logits instead of responsibilities
  const float* thr2;           // [B][N] STATS_TOPK: each row's k-th largest logit (log2)
  const int* thr_idx;          // [B][N] STATS_TOPK: its component index (ties: lower index first)
  int hard;                    // STATS_TOPK with k = 1: r = 1 for component thr_idx, else 0
  uint64_t* xch;               // STATS_XCH: [B][slices][kRing][ktiles][32] (max, tagged sum) words, set by the launcher
  unsigned* status;            // STATS_XCH: nonzero after a timed-out wait (zeroed by the launcher)
  int spin_limit;              // STATS_XCH: polls per wait (negative: give up at once)
};

// Approximate top-k EM (params.hip): per row of the (B, N, K) log2 logits, the
// k-th largest logit and its index (order: logit descending, then index
// ascending), the log-normaliser over the top k (written to lse2), and per-block
// sums of the natural-log normalisers.
void launch_topk_select(const float* logits, int B, int64_t N, int K, int top_k, float* lse2, float* thr2,
                        int* thr_idx, double* ll_part, int ll_blocks, hipStream_t s);
int topk_select_blocks(int64_t N);

int tile_cw(int cov, int dp, int bf);
int launch_tile(int cov, int bf, int dp, int mode, const TileArgs& a, dim3 grid, int nw, hipStream_t s);
// MODE_STATS_XCH (fp32 spherical / diag (DP <= 64) / tied, 8 waves): resident
// workgroups per device (0 when the instance does not exist), and the launch
// (sets the exchange words and zeroes the status first; the grid must be within
// the resident capacity, else -1); -2 when the launch fails.
int tile_xch_capacity(int cov, int dp);
int launch_tile_xch(int cov, int dp, const TileArgs& a, dim3 grid, int64_t nwords, hipStream_t s);
// Spherical bf16 kernel (em_sph_bf16.hip): dp in {32, 64} with nw in {2, 4, 8};
// dp 128 with nw 8 (and 16 for MODE_LSE).
int launch_sph_bf16(int dp, int nw, int mode, const TileArgs& a, dim3 grid, hipStream_t s);
// Fused single-pass kernel (em_fused.hip): spherical bf16, dp in {32, 64}, K <= 64;
// one wave per row slice, `slices` slices, kFusedWaves waves per workgroup. Each
// workgroup writes ONE partial statistics tile and ONE partial log-likelihood
// (index blockIdx.x; a.nslices is the number of wave slices).
constexpr int kFusedWaves = 4;
int launch_sph_bf16_fused(int dp, int k, const TileArgs& a, int slices, hipStream_t s);

// Single-pass cooperative kernel (em_coop.hip): spherical bf16 at D = 128 with
// G = ceil(K / 256) workgroups per group of rows, 2 <= G <= kMaxCoopGroup
// (256 < K <= 1024, where it measured faster than the two-pass kernels).
constexpr int kCoopComps = 256;      // components per workgroup
constexpr int kMaxCoopGroup = 4;
constexpr int kRing = 4;             // exchange slots per group
constexpr uint32_t kTagOdd = 0x80000000u;  // round-parity tag bit of an exchanged word's sum half

struct CoopArgs {
  const void* x;               // [B][N][D] bf16
  int vec_ok;
  int64_t N;
  int D, K, B;
  const void* w_mu;            // [B][K][DP] the means, bf16
  const float* w_scale;        // [B][K] log2(e)/σ²
  const void* w_aug;           // [B][K][32] bf16
  int G;                       // workgroups per group
  int NG;                      // groups (grid = NG * G)
  int spb;                     // row items per batch
  int64_t rows_per_item;       // multiple of 32
  float* part_stats;           // [spb][B][K][JP]
  double* ll_part;             // [B][spb] natural-log partial sums
  uint64_t* xch;               // [NG][kRing][G][32] exchanged (max, tagged sum) words, set by the launcher
  unsigned* status;            // nonzero after a timed-out wait (zeroed by the launcher)
  int spin_limit;
};
// Resident workgroups of the cooperative kernel on the current device.
int coop_capacity();
int launch_sph_bf16_coop(int dp, const CoopArgs& a, hipStream_t s);

// Full covariance at 16 < D <= 128 (em_full_wide.hip): whitening E-step and
// weighted-Gram statistics on split-bf16 MFMA operands (the statistics at DP = 128
// on the fp32 MFMA), DP in {32, 64, 128}.
struct FwPackArgs {
  int B, K, D, DP, prelude;
  int param_round;             // 1 bf16, 2 fp16: the prelude's normalised weights kept in that dtype
  float min_weight;
  const float* means;          // [B][K][D]
  const float* weights;        // [B][K]
  const float* linv;           // [B][K][D][D] L^-1 (lower triangular)
  const float* logdet;         // [B][K]
  void* lpack;                 // fw_lpack_bytes(B, K, DP): L^-1 as bf16 MFMA A-operand chunks (three parts)
  void* lpaug;                 // [B][K][DP/32][64][8] bf16: -L^-1 μ in three parts (lanes 0..31 of each tile)
  float4* cconst;              // [B][K] (log2 w - ½ log2(e) (D log 2π + log det), 0, 0, 0)
};
struct FwArgs {
  const float* x;              // [B][N][D] fp32
  int vec_ok;                  // D == DP and x 16-byte aligned
  int64_t N;
  int D, K, B;
  const void* lpack;
  const void* lpaug;
  const float4* cconst;
  float* l2;                   // [B][K][N] log2 logits (E-step output, statistics input), or null
  float* lse2;                 // [B][N] log2 row log-normalisers
  float* scores;               // [B][N] natural-log scores, or null
  int64_t* labels;             // [B][N] first argmax, or null
  double* ll_part;             // [B][fw_eblocks(N)] natural-log partial sums, or null
  float* part_stats;           // [slices][B][K][JP]
  int JP, nk_col;
  int64_t rows_per_slice;      // statistics kernel: rows per slice
  // Hard assignment (approximate top-k EM with k = 1): the E-step writes each
  // row's first argmax to hard_idx and its maximum as the log-normaliser; the
  // statistics take r = 1 for that component, 0 elsewhere (no logits stored).
  int hard;
  int* hard_idx;               // [B][N]
  // Approximate top-k EM with k > 1 (statistics kernel): r = 2^(l2 - lse2) for
  // the components a row keeps (logit above thr2, or equal and index <= thr_idx),
  // lse2 then being the top-k log-normaliser; 0 elsewhere.
  const float* thr2;           // [B][N] or null
  const int* thr_idx;          // [B][N]
};
int64_t fw_lpack_bytes(int B, int K, int DP);
int fw_eblocks(int64_t N);
void launch_fw_pack(const FwPackArgs& a, hipStream_t s);
// phase 0: the E-step over fw_eblocks(N) x B workgroups; 1: the statistics over
// slices x ceil(K / 4) x B.  Returns -1 for an unsupported dp.
int launch_fw(int dp, int phase, const FwArgs& a, int slices, hipStream_t s);
// proba[b][n][k] = 2^(l2[b][k][n] - lse2[b][n]), or (raw) the log2 logits l2 themselves, transposed.
void launch_fw_proba(const float* l2, const float* lse2, float* proba, int B, int64_t N, int K, hipStream_t s,
                     bool raw = false);

// Full-covariance inference at D <= 16, K <= 32 (em_full_infer.hip): whitening
// with split bf16 operands, every component of a row in one wave.
constexpr int kFull16MaxK = 32;
struct Full16Args {
  const float* x;              // [B][N][D] fp32
  int vec_ok;                  // D == 16 and x 16-byte aligned
  int64_t N;
  int D, K, B;
  const float* linv;           // pack inputs: [B][K][D][D] L^-1, means, weights (as given), log det
  const float* means;
  const float* weights;
  const float* logdet;
  void* lparts;                // [B][K][3][16][16] bf16 parts of L^-1
  float* bneg;                 // [B][K][16] -L^-1 μ
  float* c2;                   // [B][K] log2 w - ½ log2(e) (D log 2π + log det)
  float* scores;               // [B][N] natural-log scores, or null
  float* lse2;                 // [B][N] log2 log-normalisers, or null
  int64_t* labels;             // [B][N] first argmax, or null
  float* proba;                // [B][N][K] responsibilities, or null
};
void launch_full16_pack(const Full16Args& a, hipStream_t s);
void launch_full16_infer(const Full16Args& a, hipStream_t s);

// Greedy k-means++ seeding (kmeans.hip).  Row sample [B][S][D] fp32; the first
// centre's row index per batch and T uniform draws per later centre are inputs.
constexpr int kKppMaxTrials = 16;
constexpr int kKppMaxRows = 65536;
struct KppArgs {
  const float* sample;         // [B][S][D]
  int B, S, D, K, T;
  int vec;                     // rows 16-byte aligned and D % 4 == 0
  const int64_t* first;        // [B]
  const float* draws;          // [B][K-1][T] in [0, 1)
  float* centers;              // [B][K][D]
  // workspace (kpp_bind_workspace)
  float* closest;              // [B][S]
  float* dist;                 // [B][kKppMaxTrials][S]
  float* pot_part;             // [B][nblk][kKppMaxTrials]
  int* cand;                   // [B][kKppMaxTrials]
  int nblk;
};
int64_t kpp_workspace_bytes(int B, int S, int K, int T);
void kpp_bind_workspace(KppArgs& a, void* ws);
void launch_kpp(const KppArgs& a, hipStream_t s);

}  // namespace gx
