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
enum Mode { MODE_LSE = 0, MODE_STATS = 1, MODE_PROBA = 2, MODE_LSE_IDX = 3, MODE_STATS_TOPK = 4 };

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

// Index of (d, e), d <= e, in the packed upper triangle of a DP x DP matrix.
__host__ __device__ constexpr int sym_index(int d, int e, int dp) { return d * dp - d * (d - 1) / 2 + (e - d); }

__device__ __forceinline__ f32x4 mfma_bf16(bf16x8 a, bf16x8 b, f32x4 c) {
  return __builtin_amdgcn_mfma_f32_16x16x32_bf16(a, b, c, 0, 0, 0);
}
__device__ __forceinline__ f32x4 mfma_f32(float a, float b, f32x4 c) {
  return __builtin_amdgcn_mfma_f32_16x16x4f32(a, b, c, 0, 0, 0);
}

__device__ __forceinline__ float fast_exp2(float x) { return __builtin_amdgcn_exp2f(x); }

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
