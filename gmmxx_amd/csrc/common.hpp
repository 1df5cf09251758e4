// Shared device helpers for the gfx950 GMM EM engine.
#pragma once

#include <hip/hip_runtime.h>
#include <stdint.h>

namespace gx {

typedef float f32x4 __attribute__((ext_vector_type(4)));
typedef __bf16 bf16x8 __attribute__((ext_vector_type(8)));

enum Cov { SPH = 0, DIAG = 1, TIED = 2, FULL = 3 };
// MODE_STATS_TOPK: the statistics pass of approximate top-k EM -- responsibilities
// only for each row's top-k components (ranked by logit, then lower index), the
// rest zero, against the top-k log-normaliser.
// MODE_STATS_LSE / MODE_PROBA_LSE: the statistics / responsibility pass with the
// row log-normalisers formed inside the workgroup (every component is in it).
// MODE_STATS_XCH: the statistics pass with the row log-normalisers merged across
// the workgroups that hold a row slice's component tiles (exchanged partials).
enum Mode {
  MODE_LSE = 0, MODE_STATS = 1, MODE_PROBA = 2, MODE_LSE_IDX = 3, MODE_STATS_TOPK = 4, MODE_STATS_LSE = 5,
  MODE_PROBA_LSE = 6, MODE_STATS_XCH = 7
};

constexpr float kLog2e = 1.4426950408889634f;
constexpr float kLn2 = 0.6931471805599453f;
constexpr double kLog2Pi = 1.8378770664093453;  // log(2π)
constexpr int kBN = 32;                          // rows per block iteration

__host__ __device__ constexpr int round_up(int v, int m) { return (v + m - 1) / m * m; }

// Feature widths of the augmented formulation, for padded dimension DP.
//   E : E-step reduction width (columns of φ = rows of W)
//   J : M-step feature count (columns of ψ)
// Spherical/tied:  φ = x;                 diag: φ = [x² | x];  full: φ = [sym(xxᵀ) | x]
// Spherical:       ψ = [x | 1 | ‖x‖²_hi | ‖x‖²_lo]   diag: ψ = [x | x² | 1]
// Tied:            ψ = [x | 1]             full: ψ = [x | sym(xxᵀ) | 1]
template <int COV, int DP, bool BF>
struct Dims {
  static constexpr int S = DP * (DP + 1) / 2;
  static constexpr int E = (COV == SPH || COV == TIED) ? DP : (COV == DIAG ? 2 * DP : S + DP);
  static constexpr int J = (COV == SPH) ? DP + 3 : (COV == DIAG ? 2 * DP + 1 : (COV == TIED ? DP + 1 : DP + S + 1));
  static constexpr int EP = round_up(E, 32);   // whole 32-deep bf16 MFMA k-steps
  static constexpr int JP = round_up(J, 16);
  // Column of N_k in the statistics row.
  static constexpr int NK_COL = (COV == SPH) ? DP : (COV == DIAG ? 2 * DP : (COV == TIED ? DP : DP + S));
};

// Position of the product x_d·x_e (d <= e < 16) among the 136 second-order
// features of the full covariance (DP = 16), in the order the tile kernel's
// loader writes them: x is read as four 4-column chunks, one per lane of a row
// quad, and lane c owns (a) the products inside its chunk (10 per chunk, upper
// triangle row by row), (b) its chunk times chunk c+1 mod 4 (16 each, own
// column major: 4·(own) + partner), (c) for c < 2, its chunk times chunk c+2.
//   [0, 40)    diagonal chunk blocks, chunk c at 10c
//   [40, 104)  pairs {c, c+1 mod 4}, owner c at 40 + 16c ({0, 3} is owned by 3)
//   [104, 136) pairs {0, 2} and {1, 3}, owner c at 104 + 16c
__host__ __device__ constexpr int full_feature(int d, int e) {
  const int cd = d / 4, ce = e / 4, i = d % 4, j = e % 4;
  if (cd == ce) return 10 * cd + i * 4 - i * (i - 1) / 2 + (j - i);
  if (ce == cd + 1) return 40 + 16 * cd + 4 * i + j;
  if (cd == 0 && ce == 3) return 40 + 48 + 4 * j + i;
  return 104 + 16 * cd + 4 * i + j;   // ce == cd + 2
}

// Position of Σ r x_d x_e (d <= e < DP) in the statistics rows of the full
// covariance at DP >= 32: the upper triangle row by row.
__host__ __device__ constexpr int fw_tri(int DP, int d, int e) { return d * DP - d * (d - 1) / 2 + (e - d); }

// Column of Σ r x_d x_e (d <= e) after the DP columns of Σ r x in a full-covariance
// statistics row: the tile kernel's feature order at DP = 16, fw_tri above it.
__host__ __device__ constexpr int full_sxx(int DP, int d, int e) { return DP == 16 ? full_feature(d, e) : fw_tri(DP, d, e); }

__device__ __forceinline__ f32x4 mfma_bf16(bf16x8 a, bf16x8 b, f32x4 c) {
  return __builtin_amdgcn_mfma_f32_16x16x32_bf16(a, b, c, 0, 0, 0);
}
__device__ __forceinline__ f32x4 mfma_f32(float a, float b, f32x4 c) {
  return __builtin_amdgcn_mfma_f32_16x16x4f32(a, b, c, 0, 0, 0);
}

__device__ __forceinline__ float fast_exp2(float x) { return __builtin_amdgcn_exp2f(x); }
// max(v, lo) that passes a NaN v through, as torch's clamp_min does (fmaxf
// would return lo): the reference's clamps keep a non-finite input visible.
__device__ __forceinline__ float clamp_lo(float v, float lo) { return v < lo ? lo : v; }

__device__ __forceinline__ float to_f32(float v) { return v; }
__device__ __forceinline__ float to_f32(__bf16 v) { return (float)v; }

// Merge two (max, scaled-sum, argmax) triples; ties keep the smaller index.
__device__ __forceinline__ void lse_merge(float& m, float& s, int& idx, float m2, float s2, int i2) {
  float M = fmaxf(m, m2);
  float a = (m == -INFINITY) ? 0.f : s * fast_exp2(m - M);
  float b = (m2 == -INFINITY) ? 0.f : s2 * fast_exp2(m2 - M);
  bool take = (m2 > m) || (m2 == m && i2 < idx);
  idx = take ? i2 : idx;
  m = M;
  s = a + b;
}

}  // namespace gx
