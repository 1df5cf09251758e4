// Component-side kernels of one EM iteration: the iteration prelude and E-step
// operand packing, batched Cholesky with the batch-global jitter ladder,
// per-row combine of k-tile partials, ordered reductions and the M-step
// finalize for the four covariance types.  All of them touch K- or N-sized
// data only; the (N x K) work lives in em_tile.hip.

#include <math.h>

#include <hip/hip_fp16.h>

#include <algorithm>

#include "common.hpp"
#include "engine.hpp"
#include "params.hpp"

namespace gx {

// ---------------------------------------------------------------------------
// Block helpers
// ---------------------------------------------------------------------------

template <typename T>
__device__ T block_sum(T v, T* scratch) {
  // scratch: >= 32 elements of shared memory
  for (int off = 32; off >= 1; off /= 2) v += __shfl_xor(v, off);
  const int w = threadIdx.x / 64, l = threadIdx.x % 64;
  __syncthreads();
  if (l == 0) scratch[w] = v;
  __syncthreads();
  T t = 0;
  const int nw = (blockDim.x + 63) / 64;
  for (int i = 0; i < nw; ++i) t += scratch[i];  // fixed order: deterministic
  return t;
}

// Σ_k max(w_k, floor) over one batch row, identical in every block.
__device__ float weight_total(const float* w, int K, float floor_v, float* scratch) {
  float s = 0.f;
  for (int k = threadIdx.x; k < K; k += blockDim.x) s += clamp_lo(w[k], floor_v);
  return block_sum(s, scratch);
}

// ---------------------------------------------------------------------------
// Prelude + E-step operand packing (one wave per component, lanes over features)
// ---------------------------------------------------------------------------

constexpr int kMaxPrepD = 128;

__device__ __forceinline__ float wave_sum(float v) {
  for (int off = 32; off >= 1; off /= 2) v += __shfl_xor(v, off);
  return v;
}

__device__ float jitter_of(int level);

// v rounded to the parameter dtype (1 bf16, 2 fp16; 0 leaves it).
__device__ __forceinline__ float round_param(float v, int mode) {
  return mode == 1 ? (float)(__bf16)v : (mode == 2 ? (float)(__half)v : v);
}

__global__ __launch_bounds__(64) void prep_kernel(PrepArgs a) {
  __shared__ float scratch[32];
  __shared__ float mus[kMaxPrepD];
  __shared__ double fa[16][17], fp[16][17], ff[16][17];   // full covariance (D <= 16) refinement
  const int b = blockIdx.y, k = blockIdx.x, lane = threadIdx.x;
  const int K = a.K, D = a.D, DP = a.DP, EP = a.EP;
  const float* wrow = a.weights + (size_t)b * K;
  // Iteration prelude (torch_fallback.py:2061-2066): w <- max(w, min_weight) / Σ.
  // Inference uses the weights as given (log w only).
  const float floor_v = a.prelude ? a.min_weight : -INFINITY;
  const float total = a.prelude ? weight_total(wrow, K, floor_v, scratch) : 1.f;
  const size_t bk = (size_t)b * K + k;
  // (with a parameter dtype the normalised weight is kept in it, as the
  // reference's prelude divides in x's dtype)
  const float wk = a.prelude ? round_param(clamp_lo(wrow[k], floor_v) / total, a.param_round) : wrow[k];
  const float lw = logf(wk);
  const float* mu = a.means + bk * D;
  // bf16 x (spherical) computes with bf16 means, as the reference keeps them in
  // x's dtype (torch_fallback.py:2295, :1451).
  for (int d = lane; d < D; d += 64) mus[d] = a.bf ? (float)(__bf16)mu[d] : mu[d];
  __syncthreads();
  float colq, ca, cb;
  const float log2pi_d = (float)(kLog2Pi * (double)D);

  auto put_f32 = [&](int e, float v) {
    reinterpret_cast<float*>(a.w_hi)[bk * EP + e] = v;
  };
  auto put_bf = [&](int e, float v) {
    const __bf16 hi = (__bf16)v;
    reinterpret_cast<__bf16*>(a.w_hi)[bk * EP + e] = hi;
    reinterpret_cast<__bf16*>(a.w_lo)[bk * EP + e] = (__bf16)(v - (float)hi);
  };

  // fp32 x: the constant C = ca·colq + cb, which the logit adds to ca·(terms ~10²
  // times the logit), is formed in float64 (colq and cb too) and rounded once.
  double cy64 = 0.0;
  bool have64 = false;
  constexpr double kLog2eD = 1.4426950408889634;
  if (a.cov == SPH) {
    float var = a.covs[bk];
    if (a.prelude) var = clamp_lo(var, a.reg_covar);
    if (lane == 0) a.covs_used[bk] = var;
    float msq = 0.f;
    double msq64 = 0.0;
    for (int d = lane; d < D; d += 64) {
      msq = fmaf(mus[d], mus[d], msq);
      msq64 = fma((double)mus[d], (double)mus[d], msq64);
    }
    msq = wave_sum(msq);
    const float lognorm = (float)D * ((float)kLog2Pi + logf(var));
    colq = msq;
    ca = -0.5f * kLog2e / var;
    cb = (lw - 0.5f * lognorm) * kLog2e;
    if (!a.bf) {
#pragma unroll
      for (int off = 32; off >= 1; off /= 2) msq64 += __shfl_xor(msq64, off);
      const double cb64 = ((double)lw - 0.5 * (double)D * (kLog2Pi + log((double)var))) * kLog2eD;
      cy64 = (double)ca * msq64 + cb64;
      have64 = true;
    }
    if (a.bf) {
      // bf16 kernel: W' = -2·ca·μ (hi/lo) and the augmented constants
      // [A_h A_h A_h A_m A_m A_l C_h C_m | C_l 0 ...] with A = ca, C = ca·‖μ‖² + cb.
      for (int e = lane; e < EP; e += 64) put_bf(e, e < D ? -2.f * ca * mus[e] : 0.f);
      const float cy = fmaf(ca, colq, cb);
      const __bf16 ah = (__bf16)ca;
      const __bf16 am = (__bf16)(ca - (float)ah);
      const __bf16 al = (__bf16)(ca - (float)ah - (float)am);
      const __bf16 ch = (__bf16)cy;
      const __bf16 cm = (__bf16)(cy - (float)ch);
      const __bf16 cl = (__bf16)(cy - (float)ch - (float)cm);
      const __bf16 vals[9] = {ah, ah, ah, am, am, al, ch, cm, cl};
      if (lane < 32) reinterpret_cast<__bf16*>(a.w_aug)[bk * 32 + lane] = lane < 9 ? vals[lane] : (__bf16)0.f;
      // Cooperative and fused passes: the exact bf16 means and the factor -2·ca, applied to
      // the fp32 product x·μ after the MFMA (no hi/lo split of the operand).
      if (a.w_mu) {
        for (int e = lane; e < DP; e += 64) reinterpret_cast<__bf16*>(a.w_mu)[bk * DP + e] = (__bf16)(e < D ? mus[e] : 0.f);
        if (lane == 0) a.w_scale[bk] = -2.f * ca;
      }
      // Fused pass: one accumulator chain P = x·μ - ‖x‖²/2 + C' and l2 = s·P, with
      // s = -2·ca and C' = C / s = -‖μ‖²/2 + (log w - ½ D log(2πσ²))·σ² (float64,
      // from the bf16 means the product uses): [-½ -½ -½ 0 0 0 C'_h C'_m | C'_l 0 ...].
      if (a.w_augs) {
        double mb64 = 0.0;
        for (int d = lane; d < D; d += 64) {
          const double mb = (double)(float)(__bf16)mus[d];
          mb64 = fma(mb, mb, mb64);
        }
#pragma unroll
        for (int off = 32; off >= 1; off /= 2) mb64 += __shfl_xor(mb64, off);
        const double cp = -0.5 * mb64 + ((double)lw - 0.5 * (double)D * (kLog2Pi + log((double)var))) * (double)var;
        const __bf16 ph = (__bf16)(float)cp;
        const __bf16 pm = (__bf16)(float)(cp - (double)(float)ph);
        const __bf16 pl = (__bf16)(float)(cp - (double)(float)ph - (double)(float)pm);
        const __bf16 half = (__bf16)(-0.5f), zero = (__bf16)0.f;
        const __bf16 vals[9] = {half, half, half, zero, zero, zero, ph, pm, pl};
        if (lane < 16) reinterpret_cast<__bf16*>(a.w_augs)[bk * 16 + lane] = lane < 9 ? vals[lane] : zero;
      }
    } else {
      for (int e = lane; e < EP; e += 64) put_f32(e, e < D ? mus[e] : 0.f);
    }
  } else if (a.cov == DIAG) {
    // torch_fallback.py:2491-2494
    const float* vr = a.covs + bk * D;
    float* vu = a.covs_used + bk * D;
    // P = 1/v (correctly rounded either way), -2μP and Σ μ²P in float64, each
    // rounded once (fp32 chains here carried the largest share of the logit error)
    double logdet = 0.0, mpm = 0.0;
    for (int d = lane; d < D; d += 64) {
      float v = vr[d];
      if (a.prelude) v = clamp_lo(v, a.reg_covar);
      vu[d] = v;
      const float vc = clamp_lo(v, 1e-30f);
      const double p = 1.0 / (double)vc;
      const double wm = (double)mus[d] * p;
      logdet += log((double)vc);
      mpm = fma((double)mus[d], wm, mpm);
      put_f32(d, (float)p);
      put_f32(DP + d, (float)(-2.0 * wm));
    }
    for (int d = D + lane; d < DP; d += 64) { put_f32(d, 0.f); put_f32(DP + d, 0.f); }
    for (int e = 2 * DP + lane; e < EP; e += 64) put_f32(e, 0.f);
#pragma unroll
    for (int off = 32; off >= 1; off /= 2) {
      logdet += __shfl_xor(logdet, off);
      mpm += __shfl_xor(mpm, off);
    }
    colq = (float)mpm;
    ca = -0.5f * kLog2e;
    cb = (float)(((double)lw - 0.5 * ((double)log2pi_d + logdet)) * kLog2eD);
    cy64 = -0.5 * kLog2eD * mpm + ((double)lw - 0.5 * ((double)log2pi_d + logdet)) * kLog2eD;
    have64 = true;
  } else if (a.cov == TIED) {
    // Pμ_k (torch_fallback.py:2873), μᵀPμ (:2874)
    const float* P = a.prec + (size_t)b * D * D;
    double mpm = 0.0;
    for (int d = lane; d < D; d += 64) {
      double pm = 0.0;
      for (int e = 0; e < D; ++e) pm = fma((double)mus[e], (double)P[d * D + e], pm);
      mpm = fma((double)mus[d], pm, mpm);
      put_f32(d, (float)pm);
    }
    for (int e = D + lane; e < EP; e += 64) put_f32(e, 0.f);
#pragma unroll
    for (int off = 32; off >= 1; off /= 2) mpm += __shfl_xor(mpm, off);
    colq = (float)mpm;
    ca = -0.5f * kLog2e;
    cb = (lw - 0.5f * (log2pi_d + a.logdet[b])) * kLog2e;
    cy64 = (double)ca * mpm + ((double)lw - 0.5 * ((double)log2pi_d + (double)a.logdet[b])) * kLog2eD;
    have64 = true;
    if (a.shift) {
      // The tied EM logits leave out each row's xᵀPx, so the row log-normalisers
      // are each ½ xᵀPx too large; their sum, -½ Σ_n x_nᵀ P x_n = -½ Σ_rj P_rj
      // (XᵀX)_rj, is added back as D log-likelihood parts per problem, row r of
      // the trace from the blocks k ≡ r (mod K), in double.
      const float* G = a.gram + (size_t)b * D * D;
      for (int r = k; r < D; r += K) {
        double t = 0.0;
        for (int j = lane; j < D; j += 64) t = fma((double)P[r * D + j], (double)G[r * D + j], t);
#pragma unroll
        for (int off = 32; off >= 1; off /= 2) t += __shfl_xor(t, off);
        if (lane == 0) a.shift[(size_t)b * D + r] = -0.5 * t;
      }
    }
  } else {
    // FULL: W_k = [packed P_k with doubled off-diagonal | -2 P_k μ_k]  (torch_fallback.py:418-432).
    // The logit's terms reach ~10^2 times the logit, so every fp32 rounding on the
    // way to W (the inverse itself, the off-diagonal sum, the Pμ and μᵀPμ chains,
    // the constant) adds an error of that order.  The fp32 precision of the
    // Cholesky kernels (the reference's jitter ladder, torch_fallback.py:316-334)
    // is refined here by two Newton steps P <- P + P(I - A·P) in float64 against
    // A = sym(Σ) + jitter·I (formed entry by entry as the factorisation formed it),
    // which square the residual each (fp32 inverse: ~κ·1e-7), and W and the
    // constant are formed in float64 and rounded once.  A matrix the ladder left
    // unfactorised, or whose fp32 inverse is too far off (residual > 1/2),
    // keeps its fp32 precision.
    const float* P = a.prec + bk * D * D;
    const float* Cv = a.covs + bk * D * D;
    const int lv = *a.chol_level;
    const float jit = jitter_of(lv);
    for (int e = lane; e < D * D; e += 64) {
      const int r = e / D, c = e % D;
      fa[r][c] = (double)((r == c) ? Cv[r * D + c] + jit : 0.5f * (Cv[r * D + c] + Cv[c * D + r]));
      fp[r][c] = (double)P[e];
    }
    const bool refine = a.first_ok[bk] <= lv;   // D <= 16: the plan's limit for full covariance
    for (int it = 0; it < 2 && refine; ++it) {
      __syncthreads();
      double worst = 0.0;
      for (int e = lane; e < D * D; e += 64) {
        const int r = e / D, c = e % D;
        double t = (r == c) ? 1.0 : 0.0;
        for (int k = 0; k < D; ++k) t = fma(-fa[r][k], fp[k][c], t);
        ff[r][c] = t;
        worst = fmax(worst, fabs(t));
      }
#pragma unroll
      for (int off = 32; off >= 1; off /= 2) worst = fmax(worst, __shfl_xor(worst, off));
      if (!(worst <= 0.5)) break;            // whole block (one wave): keep the current P
      __syncthreads();
      double nv[4];
      for (int e = lane, u = 0; e < D * D; e += 64, ++u) {
        const int r = e / D, c = e % D;
        double t = fp[r][c];
        for (int k = 0; k < D; ++k) t = fma(fp[r][k], ff[k][c], t);
        nv[u] = t;
      }
      __syncthreads();
      for (int e = lane, u = 0; e < D * D; e += 64, ++u) fp[e / D][e % D] = nv[u];
    }
    __syncthreads();
    auto pd = [&](int d, int e) { return 0.5 * (fp[d][e] + fp[e][d]); };
    const int S = DP * (DP + 1) / 2;
    for (int e = lane; e < EP; e += 64) put_f32(e, 0.f);
    __syncthreads();   // the zero fill lands before the packed entries below
    double mpm = 0.0;
    for (int d = lane; d < D; d += 64) {
      double pm = 0.0;
      for (int e = 0; e < D; ++e) pm = fma(pd(d, e), (double)mus[e], pm);
      mpm = fma((double)mus[d], pm, mpm);
      put_f32(S + d, (float)(-2.0 * pm));
      for (int e = d; e < D; ++e) put_f32(full_feature(d, e), (float)(d == e ? pd(d, d) : pd(d, e) + pd(e, d)));
    }
#pragma unroll
    for (int off = 32; off >= 1; off /= 2) mpm += __shfl_xor(mpm, off);
    // (ca, ca·μᵀPμ + cb) with the constant rounded once from float64
    const double cbd = ((double)lw - 0.5 * ((double)log2pi_d + (double)a.logdet[bk])) * kLog2eD;
    if (lane == 0) a.cconst[bk] = make_float4(-0.5f * kLog2e, (float)(-0.5 * kLog2eD * mpm + cbd), 0.f, 0.f);
    return;
  }
  // l2 = ca * (rowq - 2S + colq) + cb (spherical, tied: S is the cross term x·μ / x·Pμ) or
  // ca * (S + colq) + cb (diag, full: W already carries the -2), stored as (ca, ca*colq + cb).
  if (lane == 0) a.cconst[bk] = make_float4(ca, have64 ? (float)cy64 : fmaf(ca, colq, cb), 0.f, 0.f);
}

// ---------------------------------------------------------------------------
// Batched Cholesky, precision and log-determinant (torch_fallback.py:316-334)
//
// chol_try:    per matrix, the first jitter level that factorises
//              (level 0 = no jitter, level i = 1e-6 * 10^(i-1), i = 1..6; 7 = none),
//              and that factor
// chol_level:  the batch-global level: the largest first level (every matrix
//              factorises there); read by chol_finish's waves themselves for
//              batches of at most kCholLevelInline matrices
// chol_finish: the factor at the global level (the stored one when it is the
//              matrix's own first level, else refactorised), X = L^-1,
//              P = XᵀX = L^-T L^-1 and log det = 2 Σ log L_jj.
// chol_one:    all three in one launch for a batch that fits one workgroup
//              (tied covariances of a few problems).
// One wave per matrix, the matrix padded to DP x DP with the identity: the
// factorisation and the inverse are blocked in 16 x 16 tiles, with the
// off-panel work (trailing updates, off-diagonal inverse blocks, P = XᵀX) on
// fp32 MFMA from per-wave LDS tiles and only the 16-wide panels' dependency
// chains on the VALU, within the wave (readlane and wavefront-scope LDS, no
// workgroup barrier).
// ---------------------------------------------------------------------------

constexpr int kMaxCholD = 64;

// The ladder is built in double and cast once, like the reference's Python float.
__device__ float jitter_of(int level) {
  double j = 0.0;
  if (level >= 1) { j = 1e-6; for (int i = 1; i < level; ++i) j *= 10.0; }
  return (float)j;
}

__device__ __forceinline__ void wave_lds_sync() {
  __builtin_amdgcn_fence(__ATOMIC_RELEASE, "wavefront");
  __builtin_amdgcn_fence(__ATOMIC_ACQUIRE, "wavefront");
}

// Row stride of the per-wave LDS tiles: 16-byte aligned rows, and lanes i and
// i + 1 four banks apart, so per-lane 16-byte row reads are conflict-free.
template <int DP>
constexpr int chol_rs() { return DP + 4; }

// Lane i's row i of sym(C) + jitter·I into registers (identity outside D x D).
// Every load is unconditional (indices clamped into the matrix, the padding
// selected afterwards), so the 2·DP loads issue back to back; the column reads
// C[c][i] are coalesced across the wave.
template <int DP>
__device__ __forceinline__ void chol_row(const float* C, int D, float jitter, float (&a)[DP]) {
  const int i = threadIdx.x & 63;
  const int ic = min(i, D - 1);
  float r[DP], t[DP];
#pragma unroll
  for (int c = 0; c < DP; ++c) {
    const int cc = min(c, D - 1);
    r[c] = C[ic * D + cc];
    t[c] = C[cc * D + ic];
  }
#pragma unroll
  for (int c = 0; c < DP; ++c) {
    const float v = (i == c) ? r[c] + jitter : 0.5f * (r[c] + t[c]);
    a[c] = (i < D && c < D) ? v : ((i == c) ? 1.f : 0.f);
  }
}

__device__ __forceinline__ float lane_val(float v, int lane) {
  return __int_as_float(__builtin_amdgcn_readlane(__float_as_int(v), lane));
}

// Per-wave LDS of the factorisation: the finished factor L and the inverse X
// (DP x chol_rs rows each, row-major) and a staging tile S (DP x kCholSRS).
constexpr int kCholSRS = 20;   // 16 panel columns + 4: 16-byte rows, lanes i and i + 1 four banks apart

template <int DP>
struct CholLds {
  float L[DP * chol_rs<DP>()];
  float X[DP * chol_rs<DP>()];
  float S[DP * kCholSRS];
};

// Waves (matrices) per workgroup: the LDS above is 40 KB per wave at DP = 64.
template <int DP>
constexpr int chol_waves() { return DP == 64 ? 2 : 4; }

__device__ __forceinline__ f32x4 mfma4(float a, float b, f32x4 c) {
  return __builtin_amdgcn_mfma_f32_16x16x4f32(a, b, c, 0, 0, 0);
}

// Blocked left-looking factorisation, panels of 16 columns (LAPACK potrf's
// blocking with potf2 on the panel).  Lane i keeps row i of A in a.  For panel
// J (columns J0..J0+15) the update A[:, J] -= L[:, <J0] · L[J, <J0]ᵀ runs on
// fp32 MFMA 16x16x4 from the finished panels in sh.L (row blocks I >= J),
// staged through sh.S back into the lanes' rows; the panel is then factorised
// in registers, left-looking within it: t_i = A_ij - Σ_{J0<=c<j} L_ic L_jc
// (row j of the panel read from lane j with readlane), L_jj = sqrt(t_j),
// L_ij = t_i · (1 / L_jj) below the diagonal, 0 above (hardware v_sqrt_f32 and
// v_rcp_f32, 1 ulp), and written to sh.L.  Returns success (every pivot > 0),
// uniform across the wave; sh.L and a hold the factor.
template <int DP>
__device__ __forceinline__ bool chol_blocked(float (&a)[DP], CholLds<DP>& sh) {
  constexpr int RS = chol_rs<DP>(), NB = DP / 16;
  const int i = threadIdx.x & 63, g = i / 16, li = i % 16;
  const int ri = min(i, DP - 1);
  bool ok = true;
#pragma unroll
  for (int J = 0; J < NB; ++J) {
    const int J0 = 16 * J;
    if (J > 0) {
#pragma unroll
      for (int I = J; I < NB; ++I) {
        const int I0 = 16 * I;
        f32x4 acc = f32x4{0.f, 0.f, 0.f, 0.f};
#pragma unroll
        for (int k0 = 0; k0 < J0; k0 += 4) acc = mfma4(sh.L[(I0 + li) * RS + k0 + g], sh.L[(J0 + li) * RS + k0 + g], acc);
        // acc[v] = (L Lᵀ)[I0 + 4g + v][J0 + li]
#pragma unroll
        for (int v = 0; v < 4; ++v) sh.S[(I0 + 4 * g + v) * kCholSRS + li] = acc[v];
      }
      wave_lds_sync();
#pragma unroll
      for (int q = 0; q < 16; q += 4) {
        const f32x4 u = *reinterpret_cast<const f32x4*>(&sh.S[ri * kCholSRS + q]);
#pragma unroll
        for (int v = 0; v < 4; ++v) a[J0 + q + v] -= (i >= J0) ? u[v] : 0.f;   // rows above: zeroed below
      }
    }
#pragma unroll
    for (int j = J0; j < J0 + 16; ++j) {
      float t[4] = {a[j], 0.f, 0.f, 0.f};
#pragma unroll
      for (int c = J0; c < j; ++c) t[c & 3] = fmaf(-a[c], lane_val(a[c], j), t[c & 3]);
      const float tj = (t[0] + t[1]) + (t[2] + t[3]);
      const float d = lane_val(tj, j);
      ok = ok && (d > 0.f);
      const float ljj = __builtin_amdgcn_sqrtf(d);
      const float inv = __builtin_amdgcn_rcpf(ljj);
      a[j] = (i < j) ? 0.f : ((i == j) ? ljj : tj * inv);
    }
    if (i < DP) {
#pragma unroll
      for (int q = 0; q < 16; q += 4)
        *reinterpret_cast<f32x4*>(&sh.L[i * RS + J0 + q]) = f32x4{a[J0 + q], a[J0 + q + 1], a[J0 + q + 2], a[J0 + q + 3]};
    }
    wave_lds_sync();
  }
  return ok;
}

// The first jitter level (0..6) at which the matrix factorises, 7 for none;
// a and sh.L hold that factor (or the last attempt).
template <int DP>
__device__ __forceinline__ int chol_first(const float* C, int D, float (&a)[DP], CholLds<DP>& sh) {
  for (int lv = 0; lv < 7; ++lv) {
    chol_row<DP>(C, D, jitter_of(lv), a);
    if (chol_blocked<DP>(a, sh)) return lv;
  }
  return 7;
}

// From the factor in sh.L: log det = 2 Σ_{i<D} log L_ii into *logdet, the
// inverse X = L^-1 into sh.X and P = XᵀX = L^-T L^-1 into Pm (D x D).
//   diagonal blocks X_GG = L_GG^-1, all four at once: lane (G, c) = (i / 16,
//     i % 16) owns column c, x_r = -(Σ_{c<=k<r} L_rk x_k) / L_rr, x_c = 1 / L_cc,
//     0 above, L_GG's rows read from sh.L (one broadcast address per group);
//   off-diagonal blocks by distance from the diagonal, on fp32 MFMA:
//     X_IJ = -X_II · Σ_{J<=K<I} L_IK X_KJ (the sum staged in sh.S);
//   P_IJ = Σ_{K>=I} X_KIᵀ X_KJ for I >= J (X is block lower triangular), each
//     entry i >= j written to both (i, j) and (j, i), so P is exactly symmetric.
template <int DP>
__device__ __forceinline__ void chol_inverse(int D, CholLds<DP>& sh, float* Pm, float* logdet, float* Xm) {
  constexpr int RS = chol_rs<DP>(), NB = DP / 16;
  const int i = threadIdx.x & 63, g = i / 16, li = i % 16;
  float ld = (i < D) ? logf(sh.L[i * RS + i]) : 0.f;
#pragma unroll
  for (int off = 32; off >= 1; off /= 2) ld += __shfl_xor(ld, off);
  if (i == 0) *logdet = 2.f * ld;
  {
    const int G0 = 16 * min(g, NB - 1), c = li;
    float x[16];
#pragma unroll
    for (int r = 0; r < 16; ++r) {
      const float* Lr = &sh.L[(G0 + r) * RS + G0];
      float t[4] = {0.f, 0.f, 0.f, 0.f};
#pragma unroll
      for (int k0 = 0; k0 < r; k0 += 4) {
        const f32x4 l4 = *reinterpret_cast<const f32x4*>(Lr + k0);
#pragma unroll
        for (int v = 0; v < 4; ++v)
          if (k0 + v < r) t[v] = fmaf(l4[v], x[k0 + v], t[v]);
      }
      const float inv = __builtin_amdgcn_rcpf(Lr[r]);
      x[r] = (r < c) ? 0.f : ((r == c) ? inv : -((t[0] + t[1]) + (t[2] + t[3])) * inv);
    }
#pragma unroll
    for (int r = 0; r < 16; ++r) sh.X[(G0 + r) * RS + G0 + c] = x[r];
  }
  wave_lds_sync();
#pragma unroll
  for (int dd = 1; dd < NB; ++dd)
#pragma unroll
    for (int J = 0; J + dd < NB; ++J) {
      const int I = J + dd, I0 = 16 * I, J0 = 16 * J;
      f32x4 acc = f32x4{0.f, 0.f, 0.f, 0.f};
#pragma unroll
      for (int k0 = J0; k0 < I0; k0 += 4) acc = mfma4(sh.L[(I0 + li) * RS + k0 + g], sh.X[(k0 + g) * RS + J0 + li], acc);
#pragma unroll
      for (int v = 0; v < 4; ++v) sh.S[(4 * g + v) * kCholSRS + li] = acc[v];
      wave_lds_sync();
      f32x4 acc2 = f32x4{0.f, 0.f, 0.f, 0.f};
#pragma unroll
      for (int k0 = 0; k0 < 16; k0 += 4) acc2 = mfma4(sh.X[(I0 + li) * RS + I0 + k0 + g], sh.S[(k0 + g) * kCholSRS + li], acc2);
#pragma unroll
      for (int v = 0; v < 4; ++v) sh.X[(I0 + 4 * g + v) * RS + J0 + li] = -acc2[v];
      wave_lds_sync();
    }
  // X itself (D x D; the blocks above the diagonal are never formed in sh.X, so
  // zeros are written there) for the whitening E-step of the full covariance at D > 16
  if (Xm)
    for (int e = i; e < D * D; e += 64) Xm[e] = (e % D <= e / D) ? sh.X[(e / D) * RS + e % D] : 0.f;
  if (!Pm) return;   // the caller needs X alone
#pragma unroll
  for (int I = 0; I < NB; ++I)
#pragma unroll
    for (int J = 0; J <= I; ++J) {
      const int I0 = 16 * I, J0 = 16 * J;
      f32x4 acc = f32x4{0.f, 0.f, 0.f, 0.f};
#pragma unroll
      for (int k0 = I0; k0 < DP; k0 += 4) acc = mfma4(sh.X[(k0 + g) * RS + I0 + li], sh.X[(k0 + g) * RS + J0 + li], acc);
      // acc[v] = P[I0 + 4g + v][J0 + li]
#pragma unroll
      for (int v = 0; v < 4; ++v) {
        const int pi = I0 + 4 * g + v, pj = J0 + li;
        if (pi >= pj && pi < D && pj < D) {
          Pm[(size_t)pi * D + pj] = acc[v];
          Pm[(size_t)pj * D + pi] = acc[v];
        }
      }
    }
}

template <int DP>
__global__ __launch_bounds__(64 * chol_waves<DP>()) void chol_try_kernel(const float* cov, int D, int M,
                                                                         int* first_ok, float* lbuf) {
  __shared__ __align__(16) CholLds<DP> sh[chol_waves<DP>()];
  const int w = threadIdx.x / 64, i = threadIdx.x & 63;
  const int m = blockIdx.x * chol_waves<DP>() + w;
  if (m >= M) return;   // whole wave
  float a[DP];
  const int level = chol_first<DP>(cov + (size_t)m * D * D, D, a, sh[w]);
  if (i == 0) first_ok[m] = level;
  if (i < DP) {
    float* Lg = lbuf + ((size_t)m * DP + i) * DP;
#pragma unroll
    for (int c = 0; c < DP; c += 4) *reinterpret_cast<f32x4*>(Lg + c) = f32x4{a[c], a[c + 1], a[c + 2], a[c + 3]};
  }
}

// Largest first level over the batch (one workgroup).
__global__ void chol_level_kernel(const int* first_ok, int M, int* level) {
  __shared__ int red[256];
  int v = 0;
  for (int m = threadIdx.x; m < M; m += blockDim.x) v = max(v, first_ok[m]);
  red[threadIdx.x] = v;
  __syncthreads();
  for (int o = blockDim.x / 2; o > 0; o /= 2) {
    if ((int)threadIdx.x < o) red[threadIdx.x] = max(red[threadIdx.x], red[threadIdx.x + o]);
    __syncthreads();
  }
  if (threadIdx.x == 0) *level = min(red[0], 6);
}

// The batch level read by each wave itself (small batches: first_ok has at
// most kCholLevelInline entries), so no separate level launch is needed.
constexpr int kCholLevelInline = 512;

__device__ int wave_level(const int* first_ok, int M) {
  int v = 0;
  for (int m = threadIdx.x & 63; m < M; m += 64) v = max(v, first_ok[m]);
#pragma unroll
  for (int off = 32; off >= 1; off /= 2) v = max(v, __shfl_xor(v, off));
  return min(v, 6);
}

// inline_level: the batch level is computed from first_ok here (M <= kCholLevelInline)
// and written to *level; otherwise read from *level.
template <int DP>
__global__ __launch_bounds__(64 * chol_waves<DP>()) void chol_finish_kernel(const float* cov, int D, int M,
                                                                            const int* first_ok, int* level,
                                                                            bool inline_level, const float* lbuf,
                                                                            float* prec, float* logdet, float* linv) {
  constexpr int RS = chol_rs<DP>();
  __shared__ __align__(16) CholLds<DP> sh[chol_waves<DP>()];
  const int w = threadIdx.x / 64, i = threadIdx.x & 63;
  const int m = blockIdx.x * chol_waves<DP>() + w;
  if (m >= M) return;   // whole wave
  const int lv = inline_level ? wave_level(first_ok, M) : *level;
  if (inline_level && m == 0 && i == 0) *level = lv;   // for readers after the launch
  if (first_ok[m] == lv) {
    if (i < DP) {
      const float* Lg = lbuf + ((size_t)m * DP + i) * DP;
#pragma unroll
      for (int c = 0; c < DP; c += 4)
        *reinterpret_cast<f32x4*>(&sh[w].L[i * RS + c]) = *reinterpret_cast<const f32x4*>(Lg + c);
    }
    wave_lds_sync();
  } else {
    float a[DP];
    chol_row<DP>(cov + (size_t)m * D * D, D, jitter_of(lv), a);
    chol_blocked<DP>(a, sh[w]);
  }
  chol_inverse<DP>(D, sh[w], prec ? prec + (size_t)m * D * D : nullptr, logdet + m,
                   linv ? linv + (size_t)m * D * D : nullptr);
}

// Whole batch in one workgroup (M <= chol_waves): factor, batch level through
// LDS, inverse, in a single launch.  first_ok and level are still written.
template <int DP>
__global__ __launch_bounds__(64 * chol_waves<DP>()) void chol_one_kernel(const float* cov, int D, int M,
                                                                         int* first_ok, int* level, float* prec,
                                                                         float* logdet, float* linv) {
  constexpr int NW = chol_waves<DP>();
  __shared__ __align__(16) CholLds<DP> sh[NW];
  __shared__ int lev[NW];
  const int w = threadIdx.x / 64, i = threadIdx.x & 63;
  const bool active = w < M;
  const float* C = cov + (size_t)w * D * D;
  float a[DP];
  int first = 0;
  if (active) first = chol_first<DP>(C, D, a, sh[w]);
  if (i == 0) {
    lev[w] = first;
    if (active) first_ok[w] = first;
  }
  __syncthreads();
  int lv = 0;
#pragma unroll
  for (int u = 0; u < NW; ++u) lv = max(lv, lev[u]);
  lv = min(lv, 6);
  if (threadIdx.x == 0) *level = lv;
  if (!active) return;   // whole wave
  if (first != lv) {
    chol_row<DP>(C, D, jitter_of(lv), a);
    chol_blocked<DP>(a, sh[w]);
  }
  chol_inverse<DP>(D, sh[w], prec ? prec + (size_t)w * D * D : nullptr, logdet + w,
                   linv ? linv + (size_t)w * D * D : nullptr);
}

// ---------------------------------------------------------------------------
// 64 < D <= 128 (tied, full): one workgroup of kChol128Threads per matrix, the
// matrix in LDS.  Unblocked right-looking factorisation (column scale, then the
// trailing update from a copy of the scaled column, two barriers per column),
// the same ladder as above: chol128_try finds each matrix's first factorising
// level and keeps that factor, chol128_finish takes it when the batch level is
// the matrix's own (else factorises at the batch level) and writes X = L^-1
// (eight lanes per column, forward substitution), P = XᵀX and 2 Σ log L_jj.  A
// wave per matrix cannot hold a 128-row panel, and these sizes are rare, so
// simplicity wins over the blocked MFMA path.
// ---------------------------------------------------------------------------

constexpr int kChol128Threads = 1024;
constexpr int kChol128RS = 129;   // row stride (floats)

// A = sym(C) + jitter·I (lower triangle) into LDS, then factorised in place;
// returns false when a pivot is not positive (or not finite).
__device__ bool chol128_factor(const float* C, int D, float jitter, float* A) {
  __shared__ float colk[128];
  const int t = threadIdx.x;
  for (int e = t; e < D * D; e += kChol128Threads) {
    const int r = e / D, c = e % D;
    if (c <= r) A[r * kChol128RS + c] = (r == c) ? C[r * D + c] + jitter : 0.5f * (C[r * D + c] + C[c * D + r]);
  }
  __syncthreads();
  for (int k = 0; k < D; ++k) {
    const float p = A[k * kChol128RS + k];
    const bool ok = p > 0.f && p < INFINITY;   // every thread reads the same pivot
    if (!ok) return false;                     // uniform over the workgroup
    const float lkk = sqrtf(p);
    const float inv = 1.f / lkk;
    __syncthreads();                           // every thread has read the pivot
    if (t == 0) A[k * kChol128RS + k] = lkk;
    for (int i = k + 1 + t; i < D; i += kChol128Threads) {
      const float v = A[i * kChol128RS + k] * inv;
      A[i * kChol128RS + k] = v;
      colk[i] = v;
    }
    __syncthreads();
    // trailing update A[i][j] -= L[i][k] L[j][k], k < j <= i: row k + 1 + t/8, columns
    // j ≡ k + 1 + t (mod 8); the column is read from colk, a separate array, so the
    // loads of one row's updates need not wait for its stores
    for (int i = k + 1 + (t >> 3); i < D; i += kChol128Threads / 8) {
      const float lik = colk[i];
      for (int j = k + 1 + (t & 7); j <= i; j += 8) A[i * kChol128RS + j] = fmaf(-lik, colk[j], A[i * kChol128RS + j]);
    }
    __syncthreads();
  }
  return true;
}

// lbuf: M x 128 x 128, the factor at the matrix's first level (lower triangle).
__global__ __launch_bounds__(kChol128Threads) void chol128_try_kernel(const float* cov, int D, int M, int* first_ok,
                                                                      float* lbuf) {
  __shared__ float A[128 * kChol128RS];
  const int m = blockIdx.x;
  if (m >= M) return;
  const float* C = cov + (size_t)m * D * D;
  int first = 7;
  for (int lv = 0; lv <= 6; ++lv) {
    if (chol128_factor(C, D, jitter_of(lv), A)) {
      first = lv;
      break;
    }
    __syncthreads();   // the failed attempt's readers are done before the next fill
  }
  if (threadIdx.x == 0) first_ok[m] = first;
  if (first < 7)
    for (int e = threadIdx.x; e < D * D; e += kChol128Threads) {
      const int r = e / D, c = e % D;
      if (c <= r) lbuf[((size_t)m * 128 + r) * 128 + c] = A[r * kChol128RS + c];
    }
}

// inline_level: the batch level is the maximum of first_ok over the batch
// (M <= kCholLevelInline), written to *level by block 0; else read from *level.
__global__ __launch_bounds__(kChol128Threads) void chol128_finish_kernel(const float* cov, int D, int M,
                                                                         const int* first_ok, int* level,
                                                                         bool inline_level, const float* lbuf,
                                                                         float* prec, float* logdet, float* linv) {
  __shared__ float A[128 * kChol128RS];
  __shared__ float X[128 * kChol128RS];
  __shared__ int lvs;
  const int m = blockIdx.x, t = threadIdx.x;
  if (m >= M) return;
  if (t == 0) {
    int v = 0;
    if (inline_level) {
      for (int i = 0; i < M; ++i) v = max(v, first_ok[i]);
      v = min(v, 6);
      if (m == 0) *level = v;
    } else {
      v = *level;
    }
    lvs = v;
  }
  __syncthreads();
  const int lv = lvs;
  if (first_ok[m] == lv) {
    // the try kernel's factor at this level
    for (int e = t; e < D * D; e += kChol128Threads) {
      const int r = e / D, c = e % D;
      if (c <= r) A[r * kChol128RS + c] = lbuf[((size_t)m * 128 + r) * 128 + c];
    }
  } else {
    // a matrix that factorises at no level keeps the partial factor, as the reference does
    (void)chol128_factor(cov + (size_t)m * D * D, D, jitter_of(lv), A);
  }
  __syncthreads();
  // X = L^-1 by forward substitution, column c owned by the eight consecutive
  // lanes 8c .. 8c+7 (one wave): lane s sums k ≡ c + s (mod 8), the eight partial
  // sums are added by a fixed xor tree, lane 0 stores X[r][c], which the group's
  // later reads see (LDS operations of one wave execute in order)
  if (t < 8 * D) {
    const int c = t >> 3, s = t & 7;
    for (int r = s; r < c; r += 8) X[r * kChol128RS + c] = 0.f;
    for (int r = c; r < D; ++r) {
      float acc = 0.f;
      for (int k = c + s; k < r; k += 8) acc = fmaf(A[r * kChol128RS + k], X[k * kChol128RS + c], acc);
      acc += __shfl_xor(acc, 1);
      acc += __shfl_xor(acc, 2);
      acc += __shfl_xor(acc, 4);
      if (s == 0) X[r * kChol128RS + c] = ((r == c) ? 1.f : -acc) / A[r * kChol128RS + r];
    }
  }
  __syncthreads();
  if (linv)
    for (int e = t; e < D * D; e += kChol128Threads) linv[(size_t)m * D * D + e] = X[(e / D) * kChol128RS + e % D];
  // P = XᵀX, entries (i >= j) mirrored: the same products in the same order on
  // both sides (skipped when the caller needs X alone)
  float* P = prec ? prec + (size_t)m * D * D : nullptr;
  for (int e = t; P && e < D * D; e += kChol128Threads) {
    const int i = e / D, j = e % D;
    if (i < j) continue;
    float acc = 0.f;
    for (int k = i; k < D; ++k) acc = fmaf(X[k * kChol128RS + i], X[k * kChol128RS + j], acc);
    P[(size_t)i * D + j] = acc;
    P[(size_t)j * D + i] = acc;
  }
  if (t < 64) {
    float ld = 0.f;
    for (int k = t; k < D; k += 64) ld += logf(A[k * kChol128RS + k]);
#pragma unroll
    for (int off = 32; off >= 1; off /= 2) ld += __shfl_xor(ld, off);
    if (t == 0) logdet[m] = 2.f * ld;
  }
}

// ---------------------------------------------------------------------------
// Tied: per-row quadratic form xᵀ P x (torch_fallback.py:451)
// ---------------------------------------------------------------------------

// One thread per row; P staged in LDS, zero-padded to DP x DP so the unrolled
// loops need no bounds (all lanes read the same P entry: LDS broadcast).
// q = Σ_d x_d (P_dd x_d + 2 Σ_{e>d} P_de x_e), P symmetric.
template <int DP>
__global__ __launch_bounds__(256) void rowquad_kernel(const float* __restrict__ x, int64_t N, int D,
                                                      const float* __restrict__ prec, float* __restrict__ rowq) {
  __shared__ float Ps[DP * DP];
  const int b = blockIdx.y;
  const float* P = prec + (size_t)b * D * D;
  for (int i = threadIdx.x; i < DP * DP; i += blockDim.x) {
    const int r = i / DP, c = i % DP;
    Ps[i] = (r < D && c < D) ? P[r * D + c] : 0.f;
  }
  __syncthreads();
  const int64_t n = (int64_t)blockIdx.x * blockDim.x + threadIdx.x;
  if (n >= N) return;
  const float* xr = x + ((size_t)b * N + n) * D;
  float xv[DP];
#pragma unroll
  for (int d = 0; d < DP; ++d) xv[d] = d < D ? xr[d] : 0.f;
  float q = 0.f;
#pragma unroll
  for (int d = 0; d < DP; ++d) {
    float t = 0.5f * Ps[d * DP + d] * xv[d];
#pragma unroll
    for (int e = d + 1; e < DP; ++e) t = fmaf(Ps[d * DP + e], xv[e], t);
    q = fmaf(xv[d], t, q);
  }
  rowq[(size_t)b * N + n] = 2.f * q;
}

// ---------------------------------------------------------------------------
// Per-row combine of k-tile partials: log-normaliser, first argmax, Σ lse
// ---------------------------------------------------------------------------

__global__ void combine_kernel(CombineArgs a) {
  __shared__ double scratch[32];
  const int b = blockIdx.y;
  const int64_t n = (int64_t)blockIdx.x * blockDim.x + threadIdx.x;
  double contrib = 0.0;
  if (n < a.N) {
    float m = -INFINITY, s = 0.f;
    int idx = 0x7fffffff;
    for (int t = 0; t < a.ktiles; ++t) {
      const size_t o = ((size_t)t * a.B + b) * a.N + n;
      // Argmax partials exist only when the tile pass tracked them (labels requested).
      lse_merge(m, s, idx, a.part_ms[2 * o], a.part_ms[2 * o + 1], (a.labels || a.idx32) ? a.part_idx[o] : 0);
    }
    const float lse2 = a.max_only ? m : m + __log2f(s);
    const size_t o = (size_t)b * a.N + n;
    if (a.lse2) a.lse2[o] = lse2;
    const float lse = lse2 * kLn2;
    if (a.scores) a.scores[o] = lse;
    if (a.labels) a.labels[o] = (int64_t)idx;
    if (a.idx32) a.idx32[o] = idx;
    contrib = (double)lse;
  }
  const double t = block_sum(contrib, scratch);
  if (threadIdx.x == 0 && a.ll_part) a.ll_part[(size_t)b * gridDim.x + blockIdx.x] = t;
}

// ---------------------------------------------------------------------------
// Approximate top-k EM: per-row top-k selection over the materialised logits
// (torch_fallback.py:667-716 _topk_logits_for_chunk, :719-777 _accumulate_topk_stats)
// ---------------------------------------------------------------------------

constexpr int kSelWaves = 4;   // rows (waves) per block

int topk_select_blocks(int64_t N) { return (int)((N + kSelWaves - 1) / kSelWaves); }

// One wave per row.  Round j finds the largest logit that comes after round
// j-1's pick in the order (logit descending, index ascending): a lane scans
// its strided share of the row, then the wave reduces (max logit, min index).
// After top_k rounds: threshold = the k-th pick, lse2 = m + log2 Σ_j 2^(v_j - m)
// over the picks (m = the first); the block sums lse2·ln2 in a fixed order.
__global__ __launch_bounds__(64 * kSelWaves) void topk_select_kernel(const float* __restrict__ logits, int64_t N,
                                                                     int K, int top_k, float* lse2, float* thr2,
                                                                     int* thr_idx, double* ll_part) {
  __shared__ double llw[kSelWaves];
  const int b = blockIdx.y, wave = threadIdx.x / 64, lane = threadIdx.x % 64;
  const int64_t n = (int64_t)blockIdx.x * kSelWaves + wave;
  double contrib = 0.0;
  if (n < N) {
    const float* row = logits + ((size_t)b * N + n) * K;
    float pv = INFINITY;   // previous pick (value, index)
    int pi = -1;
    float m = 0.f, sum = 0.f;
    for (int j = 0; j < top_k; ++j) {
      float bv = -INFINITY;
      int bi = 0x7fffffff;
      for (int k = lane; k < K; k += 64) {
        const float v = row[k];
        const bool after = v < pv || (v == pv && k > pi);
        if (after && (v > bv || (v == bv && k < bi))) { bv = v; bi = k; }
      }
      for (int off = 32; off >= 1; off /= 2) {
        const float ov = __shfl_xor(bv, off);
        const int oi = __shfl_xor(bi, off);
        if (ov > bv || (ov == bv && oi < bi)) { bv = ov; bi = oi; }
      }
      if (j == 0) m = bv;
      sum += fast_exp2(bv - m);
      pv = bv;
      pi = bi;
    }
    const float l2 = m + __log2f(sum);
    if (lane == 0) {
      const size_t o = (size_t)b * N + n;
      lse2[o] = l2;
      thr2[o] = pv;
      thr_idx[o] = pi;
    }
    contrib = (double)l2 * (double)kLn2;
  }
  if (lane == 0) llw[wave] = contrib;
  __syncthreads();
  if (threadIdx.x == 0) {
    double t = 0.0;
    for (int w = 0; w < kSelWaves; ++w) t += llw[w];
    ll_part[(size_t)b * gridDim.x + blockIdx.x] = t;
  }
}

// The same selection with the row held in registers (NV values per lane,
// K <= 64·NV): the row is read once instead of once per round.
template <int NV>
__global__ __launch_bounds__(64 * kSelWaves) void topk_select_reg_kernel(const float* __restrict__ logits,
                                                                         int64_t N, int K, int top_k, float* lse2,
                                                                         float* thr2, int* thr_idx, double* ll_part) {
  __shared__ double llw[kSelWaves];
  const int b = blockIdx.y, wave = threadIdx.x / 64, lane = threadIdx.x % 64;
  const int64_t n = (int64_t)blockIdx.x * kSelWaves + wave;
  double contrib = 0.0;
  if (n < N) {
    const float* row = logits + ((size_t)b * N + n) * K;
    float v[NV];
#pragma unroll
    for (int j = 0; j < NV; ++j) v[j] = (lane + 64 * j < K) ? row[lane + 64 * j] : -INFINITY;
    float pv = INFINITY;   // previous pick (value, index)
    int pi = -1;
    float m = 0.f, sum = 0.f;
    for (int r = 0; r < top_k; ++r) {
      float bv = -INFINITY;
      int bi = 0x7fffffff;
#pragma unroll
      for (int j = 0; j < NV; ++j) {
        const int k = lane + 64 * j;
        const bool after = v[j] < pv || (v[j] == pv && k > pi);
        if (k < K && after && (v[j] > bv || (v[j] == bv && k < bi))) { bv = v[j]; bi = k; }
      }
      for (int off = 32; off >= 1; off /= 2) {
        const float ov = __shfl_xor(bv, off);
        const int oi = __shfl_xor(bi, off);
        if (ov > bv || (ov == bv && oi < bi)) { bv = ov; bi = oi; }
      }
      if (r == 0) m = bv;
      sum += fast_exp2(bv - m);
      pv = bv;
      pi = bi;
    }
    const float l2 = m + __log2f(sum);
    if (lane == 0) {
      const size_t o = (size_t)b * N + n;
      lse2[o] = l2;
      thr2[o] = pv;
      thr_idx[o] = pi;
    }
    contrib = (double)l2 * (double)kLn2;
  }
  if (lane == 0) llw[wave] = contrib;
  __syncthreads();
  if (threadIdx.x == 0) {
    double t = 0.0;
    for (int w = 0; w < kSelWaves; ++w) t += llw[w];
    ll_part[(size_t)b * gridDim.x + blockIdx.x] = t;
  }
}

void launch_topk_select(const float* logits, int B, int64_t N, int K, int top_k, float* lse2, float* thr2,
                        int* thr_idx, double* ll_part, int ll_blocks, hipStream_t s) {
  const dim3 grid(ll_blocks, B), block(64 * kSelWaves);
  if (K <= 64 * 4)
    topk_select_reg_kernel<4><<<grid, block, 0, s>>>(logits, N, K, top_k, lse2, thr2, thr_idx, ll_part);
  else if (K <= 64 * 16)
    topk_select_reg_kernel<16><<<grid, block, 0, s>>>(logits, N, K, top_k, lse2, thr2, thr_idx, ll_part);
  else if (K <= 64 * 64)
    topk_select_reg_kernel<64><<<grid, block, 0, s>>>(logits, N, K, top_k, lse2, thr2, thr_idx, ll_part);
  else
    topk_select_kernel<<<grid, block, 0, s>>>(logits, N, K, top_k, lse2, thr2, thr_idx, ll_part);
}


// Mean log-likelihood over all B*N rows (lower bound of the iteration).
__global__ void ll_reduce_kernel(const double* ll_part, int count, double inv_total, float* out) {
  __shared__ double scratch[32];
  double s = 0.0;
  for (int i = threadIdx.x; i < count; i += blockDim.x) s += ll_part[i];
  s = block_sum(s, scratch);
  if (threadIdx.x == 0) out[0] = (float)(s * inv_total);
}

// out[i] = Σ_s part[s * M + i] in a fixed order (deterministic): a block owns
// 64 outputs; wave g sums slices g, g + 16, ...; the 16 wave sums are then
// added in wave order.
constexpr int kRedWaves = 16;
// blockIdx.y selects a group of `per` consecutive slices (written to out + y*M).
// ll.out != null: the grid has one more workgroup (the last), which does the
// log-likelihood reduction of LlFold instead.
__global__ __launch_bounds__(64 * kRedWaves) void reduce_slices_kernel(const float* part, int slices, int64_t M,
                                                                       float* out, int per, LlFold ll) {
  __shared__ float red[kRedWaves][64];
  if (ll.out && blockIdx.x == gridDim.x - 1) {
    __shared__ double scratch[32];
    double t = 0.0;
    for (int i = threadIdx.x; i < ll.count; i += blockDim.x) t += ll.part[i];
    t = block_sum(t, scratch);
    if (threadIdx.x == 0) {
      float v = (float)(t * ll.inv_total);
      if (ll.status && *ll.status != 0u) {
        v = __builtin_nanf("");
        *ll.sticky |= *ll.status;
      }
      ll.out[0] = v;
    }
    return;
  }
  const int lane = threadIdx.x & 63, g = threadIdx.x >> 6;
  const int64_t i = (int64_t)blockIdx.x * 64 + lane;
  part += (size_t)blockIdx.y * per * M;
  out += (size_t)blockIdx.y * M;
  slices = min(per, slices - (int)blockIdx.y * per);
  float s = 0.f;
  if (i < M)
    for (int t = g; t < slices; t += kRedWaves) s += part[(size_t)t * M + i];
  red[g][lane] = s;
  __syncthreads();
  if (g == 0 && i < M) {
    float tot = red[0][lane];
    for (int w = 1; w < kRedWaves; ++w) tot += red[w][lane];
    out[i] = tot;
  }
}

// ---------------------------------------------------------------------------
// M-step finalize (one thread per component; weights renormalised per batch)
// spherical torch_fallback.py:2293-2305, diag :2654-2666, tied/full means :3143-3146
// ---------------------------------------------------------------------------

// Σ_k max(N_k / N, min_weight) of batch b, identical in every block.
__device__ float finalize_total(const FinalizeArgs& a, int b, float* scratch) {
  const float* st = a.stats + (size_t)b * a.K * a.JP + a.nk_col;
  float part = 0.f;
  for (int k = threadIdx.x; k < a.K; k += blockDim.x) part += clamp_lo(st[(size_t)k * a.JP] / (float)a.N, a.min_weight);
  return block_sum(part, scratch);
}

// Component k of batch b, one wave (lanes over the features): w_new =
// max(N_k / N, min_weight) / total (torch_fallback.py:2303-2305); means and
// spherical/diag variances with the active mask (:2293-2302, :2654-2666).
__device__ void finalize_comp(const FinalizeArgs& a, int b, int k, float total) {
  const int lane = threadIdx.x & 63;
  const int D = a.D;
  const size_t bk = (size_t)b * a.K + k;
  const float* sk = a.stats + bk * a.JP;
  const float nk = sk[a.nk_col];
  const bool active = nk > a.min_weight;
  const float nk_safe = clamp_lo(nk, a.min_weight);
  float* mu = a.means + bk * D;
  float msq = 0.f;
  for (int d = lane; d < D; d += 64) {
    const float m = active ? sk[d] / nk_safe : mu[d];
    // bf16 x: the means are stored in bf16 (torch_fallback.py:2295); the spherical
    // variance below is formed from the unrounded mean.  A parameter dtype rounds
    // the means (and the diag variances, formed from the rounded means as
    // :2654-2666 does) to it.
    const float mr = a.bf_means ? (float)(__bf16)m : round_param(m, a.param_round);
    mu[d] = mr;
    msq = fmaf(m, m, msq);
    if (a.cov == DIAG) {
      const float v = clamp_lo(sk[a.DP + d] / nk_safe - mr * mr, a.reg_covar);
      a.covs[bk * D + d] = active ? round_param(v, a.param_round) : a.covs_used[bk * D + d];
    }
  }
  if (a.cov == SPH) {
    for (int off = 32; off >= 1; off /= 2) msq += __shfl_xor(msq, off);
    float sq = 0.f;
    for (int i = 0; i < a.sq_n; ++i) sq += sk[a.sq_col + i];
    float v = clamp_lo(sq - nk * msq, 0.f) / (nk_safe * (float)D);
    v = clamp_lo(v, a.reg_covar);
    if (lane == 0) a.covs[bk] = active ? v : a.covs_used[bk];
  }
  if (lane == 0) {
    const float wn = clamp_lo(nk / (float)a.N, a.min_weight) / total;
    a.weights[bk] = a.cov == SPH ? wn : round_param(wn, a.param_round);   // (spherical weights stay fp32)
  }
}

// One wave per component, kFinWaves components per block.
constexpr int kFinWaves = 4;
__global__ __launch_bounds__(64 * kFinWaves) void finalize_kernel(FinalizeArgs a) {
  __shared__ float scratch[32];
  if (a.skip && *a.skip != 0u) return;   // uniform across the launch
  const int b = blockIdx.y;
  const float total = finalize_total(a, b, scratch);
  const int k = blockIdx.x * kFinWaves + threadIdx.x / 64;
  if (k < a.K) finalize_comp(a, b, k, total);
}

// Tied: Σ = sym((XᵀX − Σ_k n_k μ_k μ_kᵀ) / N) + reg·I   (torch_fallback.py:3159-3162)
// One block per (row d, batch b), one thread per column e; four partial sums
// over the components keep the loads in flight.  s_de is formed with the same
// products in the same order for (d, e) and (e, d), so the result is symmetric.
constexpr int kTiedWaves = 4;   // waves per covariance row, splitting the components

__global__ __launch_bounds__(64 * kTiedWaves) void finalize_tied_kernel(FinalizeArgs a) {
  __shared__ float red[kTiedWaves][64];
  // column e of row d; blockIdx.z picks the half of the columns (D > 64)
  const int b = blockIdx.y, d = blockIdx.x, w = threadIdx.x / 64, e = (threadIdx.x & 63) + 64 * blockIdx.z;
  if (a.skip && *a.skip != 0u) return;   // uniform over the grid
  const int K = a.K, D = a.D, JP = a.JP;
  const int ec = min(e, D - 1);
  const float* st = a.stats + (size_t)b * K * JP + a.nk_col;
  const float* mu = a.means + (size_t)b * K * D;
  // Σ_k N_k μ_kd μ_ke over k ≡ w (mod kTiedWaves), four chains
  float s0 = 0.f, s1 = 0.f, s2 = 0.f, s3 = 0.f;
  int k = w;
  for (; k + 3 * kTiedWaves < K; k += 4 * kTiedWaves) {
    s0 = fmaf(st[(size_t)k * JP], mu[k * D + d] * mu[k * D + ec], s0);
    s1 = fmaf(st[(size_t)(k + 4) * JP], mu[(k + 4) * D + d] * mu[(k + 4) * D + ec], s1);
    s2 = fmaf(st[(size_t)(k + 8) * JP], mu[(k + 8) * D + d] * mu[(k + 8) * D + ec], s2);
    s3 = fmaf(st[(size_t)(k + 12) * JP], mu[(k + 12) * D + d] * mu[(k + 12) * D + ec], s3);
  }
  for (; k < K; k += kTiedWaves) s0 = fmaf(st[(size_t)k * JP], mu[k * D + d] * mu[k * D + ec], s0);
  const int el = threadIdx.x & 63;
  red[w][el] = (s0 + s1) + (s2 + s3);
  __syncthreads();
  if (w != 0 || e >= D) return;
  const float sde = (red[0][el] + red[1][el]) + (red[2][el] + red[3][el]);
  const float* G = a.gram + (size_t)b * D * D;
  const float ade = (G[d * D + e] - sde) / (float)a.N;
  const float aed = (G[e * D + d] - sde) / (float)a.N;
  a.covs[(size_t)b * D * D + d * D + e] = round_param(0.5f * (ade + aed) + (d == e ? a.reg_covar : 0.f), a.param_round);
}

// Full: Σ_k = sym((Σ r xxᵀ − n_k μμᵀ) / max(n_k, floor)) + reg·I, kept if inactive (:3150-3158)
__global__ void finalize_full_kernel(FinalizeArgs a) {
  const int b = blockIdx.y, k = blockIdx.x;
  const int K = a.K, D = a.D, JP = a.JP, DP = a.DP;
  if (a.skip && *a.skip != 0u) return;
  const size_t bk = (size_t)b * K + k;
  const float* sk = a.stats + bk * JP;
  const float nk = sk[a.nk_col];
  const bool active = nk > a.min_weight;
  const float nk_safe = clamp_lo(nk, a.min_weight);
  const float* mu = a.means + bk * D;
  float* C = a.covs + bk * D * D;
  for (int t = threadIdx.x; t < D * D; t += blockDim.x) {
    const int d = t / D, e = t % D;
    const float sxx = sk[DP + full_sxx(DP, d < e ? d : e, d < e ? e : d)];
    const float ade = (sxx - nk * (mu[d] * mu[e])) / nk_safe;
    const float aed = (sxx - nk * (mu[e] * mu[d])) / nk_safe;
    const float v = 0.5f * (ade + aed) + (d == e ? a.reg_covar : 0.f);
    if (active) C[t] = round_param(v, a.param_round);  // inactive components keep their previous covariance
  }
}

// Unpacks the statistics rows into (N_k, Σ r x, Σ r q(x)) for callers and tests.
__global__ void unpack_stats_kernel(UnpackArgs a) {
  const int b = blockIdx.y;
  const int k = blockIdx.x * blockDim.x + threadIdx.x;
  if (k >= a.K) return;
  const size_t bk = (size_t)b * a.K + k;
  const float* sk = a.stats + bk * a.JP;
  const int D = a.D, DP = a.DP;
  a.nk[bk] = sk[a.nk_col];
  for (int d = 0; d < D; ++d) a.sum_x[bk * D + d] = sk[d];
  if (!a.sum_q) return;
  if (a.cov == SPH) {
    float sq = 0.f;
    for (int i = 0; i < a.sq_n; ++i) sq += sk[a.sq_col + i];
    a.sum_q[bk] = sq;
  } else if (a.cov == DIAG) {
    for (int d = 0; d < D; ++d) a.sum_q[bk * D + d] = sk[DP + d];
  } else if (a.cov == FULL) {
    for (int d = 0; d < D; ++d)
      for (int e = 0; e < D; ++e)
        a.sum_q[(bk * D + d) * D + e] = sk[DP + full_sxx(DP, d < e ? d : e, d < e ? e : d)];
  }
}

// Packs caller statistics into the rows the finalize kernels read (one thread per
// component); the spherical Σ r‖x‖² goes to the first of the sq columns.
__global__ void pack_stats_kernel(PackArgs a) {
  const int b = blockIdx.y;
  const int k = blockIdx.x * blockDim.x + threadIdx.x;
  if (k >= a.K) return;
  const size_t bk = (size_t)b * a.K + k;
  float* sk = a.stats + bk * a.JP;
  const int D = a.D, DP = a.DP;
  for (int j = 0; j < a.JP; ++j) sk[j] = 0.f;
  sk[a.nk_col] = a.nk[bk];
  for (int d = 0; d < D; ++d) sk[d] = a.sum_x[bk * D + d];
  if (a.cov == SPH) {
    sk[a.sq_col] = a.sum_q[bk];
    a.covs_used[bk] = clamp_lo(a.covs[bk], a.reg_covar);
  } else if (a.cov == DIAG) {
    for (int d = 0; d < D; ++d) {
      sk[DP + d] = a.sum_q[bk * D + d];
      a.covs_used[bk * D + d] = clamp_lo(a.covs[bk * D + d], a.reg_covar);
    }
  } else if (a.cov == FULL) {
    for (int d = 0; d < D; ++d)
      for (int e = d; e < D; ++e) sk[DP + full_sxx(DP, d, e)] = a.sum_q[(bk * D + d) * D + e];
  }
}

// ---------------------------------------------------------------------------
// XᵀX per batch (tied, once per fit; torch_fallback.py:2856-2862)
// ---------------------------------------------------------------------------

// One workgroup per (row slice, batch), kGramWaves waves over consecutive row
// quarters of the slice.  Four rows at a time feed T x T fp32 MFMAs
// (v_mfma_f32_16x16x4f32): lane (i, g) loads x[n + g][16t + i] for each 16-column
// tile t, which is both the A fragment (Xᵀ) and the B fragment (X) of the tile
// pairs; the accumulator of tiles (ti, tj) holds G[16ti + 4g + v][16tj + i].
// The waves' sums meet in LDS and the workgroup writes one partial.
constexpr int kGramWaves = 4;

// D > 64: blockIdx.z = 2·qi + qj picks the 64 x 64 quadrant (rows 64qi.., columns
// 64qj..) of G that the workgroup sums, with T = 4.
template <int T>
__global__ __launch_bounds__(64 * kGramWaves) void gram_mfma_kernel(const float* x, int64_t N, int D,
                                                                    int64_t rows_per_slice, float* part) {
  constexpr int DPG = 16 * T;
  __shared__ float red[kGramWaves][DPG * DPG];
  const int b = blockIdx.y, slice = blockIdx.x;
  const int orow = DPG * (blockIdx.z >> 1), ocol = DPG * (blockIdx.z & 1);
  const int w = threadIdx.x / 64, lane = threadIdx.x & 63, li = lane & 15, g = lane >> 4;
  const int64_t r0 = (int64_t)slice * rows_per_slice;
  const int64_t r1 = (r0 + rows_per_slice < N) ? r0 + rows_per_slice : N;
  const int64_t q = rows_per_slice / kGramWaves;             // multiple of 4
  const int64_t w0 = r0 + w * q;
  const int64_t w1 = (w0 + q < r1) ? w0 + q : r1;
  const float* xb = x + (size_t)b * N * D;
  f32x4 acc[T][T];
#pragma unroll
  for (int ti = 0; ti < T; ++ti)
#pragma unroll
    for (int tj = 0; tj < T; ++tj) acc[ti][tj] = f32x4{0.f, 0.f, 0.f, 0.f};
  for (int64_t n = w0; n < w1; n += 4) {
    const int64_t row = n + g;
    float f[T], fc[T];
#pragma unroll
    for (int t = 0; t < T; ++t) {
      const int c = orow + 16 * t + li, cc = ocol + 16 * t + li;
      f[t] = (row < w1 && c < D) ? xb[(size_t)row * D + c] : 0.f;
      fc[t] = (row < w1 && cc < D) ? xb[(size_t)row * D + cc] : 0.f;
    }
#pragma unroll
    for (int ti = 0; ti < T; ++ti)
#pragma unroll
      for (int tj = 0; tj < T; ++tj) acc[ti][tj] = mfma_f32(f[ti], fc[tj], acc[ti][tj]);
  }
#pragma unroll
  for (int ti = 0; ti < T; ++ti)
#pragma unroll
    for (int tj = 0; tj < T; ++tj)
#pragma unroll
      for (int v = 0; v < 4; ++v) red[w][(16 * ti + 4 * g + v) * DPG + 16 * tj + li] = acc[ti][tj][v];
  __syncthreads();
  float* out = part + ((size_t)slice * gridDim.y + b) * D * D;
  for (int o = threadIdx.x; o < DPG * DPG; o += blockDim.x) {
    const int dl = o / DPG, el = o % DPG, d = orow + dl, e = ocol + el;
    if (d >= D || e >= D) continue;
    float sum = 0.f;
#pragma unroll
    for (int u = 0; u < kGramWaves; ++u) sum += red[u][dl * DPG + el];
    out[(size_t)d * D + e] = sum;
  }
}

__global__ void canary_kernel(const int32_t* in, int32_t* out, int64_t n, int32_t offset) {
  const int64_t i = (int64_t)blockIdx.x * blockDim.x + threadIdx.x;
  if (i < n) out[i] = in[i] + offset;
}

}  // namespace gx

// ---------------------------------------------------------------------------
// Host launchers
// ---------------------------------------------------------------------------

namespace gx {

void launch_prep(const PrepArgs& a, hipStream_t s) {
  prep_kernel<<<dim3(a.K, a.B), 64, 0, s>>>(a);
}


int chol_dp(int D) { return D <= 16 ? 16 : (D <= 32 ? 32 : (D <= 64 ? 64 : 128)); }

template <int DP>
static void launch_chol_dp(const float* cov, int D, int M, int* first_ok, int* level, float* lbuf, float* prec,
                           float* logdet, float* linv, hipStream_t s) {
  constexpr int NW = chol_waves<DP>();
  if (M <= NW) {
    chol_one_kernel<DP><<<1, 64 * NW, 0, s>>>(cov, D, M, first_ok, level, prec, logdet, linv);
    return;
  }
  const int blocks = (M + NW - 1) / NW;
  chol_try_kernel<DP><<<blocks, 64 * NW, 0, s>>>(cov, D, M, first_ok, lbuf);
  const bool inline_level = M <= kCholLevelInline;
  if (!inline_level) chol_level_kernel<<<1, 256, 0, s>>>(first_ok, M, level);
  chol_finish_kernel<DP><<<blocks, 64 * NW, 0, s>>>(cov, D, M, first_ok, level, inline_level, lbuf, prec,
                                                    logdet, linv);
}

void launch_chol(const float* cov, int D, int M, int* first_ok, int* level, float* lbuf, float* prec,
                 float* logdet, hipStream_t s, float* linv) {
  if (D > 64) {
    if (M <= 0) return;
    chol128_try_kernel<<<M, kChol128Threads, 0, s>>>(cov, D, M, first_ok, lbuf);
    const bool inline_level = M <= kCholLevelInline;
    if (!inline_level) chol_level_kernel<<<1, 256, 0, s>>>(first_ok, M, level);
    chol128_finish_kernel<<<M, kChol128Threads, 0, s>>>(cov, D, M, first_ok, level, inline_level, lbuf, prec,
                                                        logdet, linv);
    return;
  }
  switch (chol_dp(D)) {
    case 16: launch_chol_dp<16>(cov, D, M, first_ok, level, lbuf, prec, logdet, linv, s); break;
    case 32: launch_chol_dp<32>(cov, D, M, first_ok, level, lbuf, prec, logdet, linv, s); break;
    default: launch_chol_dp<64>(cov, D, M, first_ok, level, lbuf, prec, logdet, linv, s); break;
  }
}

void launch_rowquad(const float* x, int B, int64_t N, int D, const float* prec, float* rowq, hipStream_t s) {
  dim3 grid((unsigned)((N + 255) / 256), B);
  if (D <= 16)
    rowquad_kernel<16><<<grid, 256, 0, s>>>(x, N, D, prec, rowq);
  else if (D <= 32)
    rowquad_kernel<32><<<grid, 256, 0, s>>>(x, N, D, prec, rowq);
  else if (D <= 64)
    rowquad_kernel<64><<<grid, 256, 0, s>>>(x, N, D, prec, rowq);
  else
    rowquad_kernel<128><<<grid, 256, 0, s>>>(x, N, D, prec, rowq);
}

int combine_blocks(int64_t N) { return (int)((N + 255) / 256); }

int launch_combine(const CombineArgs& a, hipStream_t s) {
  const int nb = combine_blocks(a.N);
  combine_kernel<<<dim3(nb, a.B), 256, 0, s>>>(a);
  return nb;
}

void launch_ll_reduce(const double* ll_part, int count, double inv_total, float* out, hipStream_t s) {
  ll_reduce_kernel<<<1, 1024, 0, s>>>(ll_part, count, inv_total, out);
}

void launch_reduce_slices(const float* part, int slices, int64_t M, float* out, hipStream_t s, float* tmp,
                          int64_t tmp_floats, const LlFold* ll) {
  // Many slices over few outputs: first sum groups of slices in parallel into
  // tmp (fixed grouping, so the result stays deterministic), then the groups.
  const int64_t blocks = (M + 63) / 64;
  int groups = 1;
  while (groups < 64 && blocks * groups < 512 && slices / (2 * groups) >= 4 * kRedWaves &&
         (int64_t)(2 * groups) * M <= tmp_floats)
    groups *= 2;
  const LlFold none{};
  const LlFold lf = ll ? *ll : none;
  const unsigned last = (unsigned)blocks + (ll ? 1u : 0u);
  if (groups == 1 || !tmp) {
    reduce_slices_kernel<<<last, 64 * kRedWaves, 0, s>>>(part, slices, M, out, slices, lf);
    return;
  }
  const int per = (slices + groups - 1) / groups;
  groups = (slices + per - 1) / per;  // every group non-empty
  reduce_slices_kernel<<<dim3((unsigned)blocks, groups), 64 * kRedWaves, 0, s>>>(part, slices, M, tmp, per, none);
  reduce_slices_kernel<<<last, 64 * kRedWaves, 0, s>>>(tmp, groups, M, out, groups, lf);
}

__global__ void take_status_kernel(unsigned* sticky, uint32_t* out) {
  if (threadIdx.x == 0) {
    *out = *sticky;
    *sticky = 0u;
  }
}

__global__ void zero_words_kernel(unsigned* p, int n) {
  const int i = blockIdx.x * blockDim.x + threadIdx.x;
  if (i < n) p[i] = 0u;
}

void launch_zero_words(unsigned* p, int n, hipStream_t s) {
  zero_words_kernel<<<(n + 255) / 256, 256, 0, s>>>(p, n);
}

void launch_take_status(unsigned* sticky, uint32_t* out, hipStream_t s) {
  take_status_kernel<<<1, 64, 0, s>>>(sticky, out);
}

void launch_finalize(const FinalizeArgs& a, hipStream_t s) {
  finalize_kernel<<<dim3((a.K + kFinWaves - 1) / kFinWaves, a.B), 64 * kFinWaves, 0, s>>>(a);
  if (a.cov == TIED) finalize_tied_kernel<<<dim3(a.D, a.B, (a.D + 63) / 64), 64 * kTiedWaves, 0, s>>>(a);
  if (a.cov == FULL) finalize_full_kernel<<<dim3(a.K, a.B), 256, 0, s>>>(a);
}

void launch_unpack(const UnpackArgs& a, int B, hipStream_t s) {
  unpack_stats_kernel<<<dim3((a.K + 255) / 256, B), 256, 0, s>>>(a);
}

void launch_pack(const PackArgs& a, int B, hipStream_t s) {
  pack_stats_kernel<<<dim3((a.K + 255) / 256, B), 256, 0, s>>>(a);
}

void launch_gram(const float* x, int B, int64_t N, int D, int slices, int64_t rows_per_slice, float* part,
                 hipStream_t s) {
  const dim3 grid(slices, B, D > 64 ? 4 : 1), block(64 * kGramWaves);
  if (D <= 16) gram_mfma_kernel<1><<<grid, block, 0, s>>>(x, N, D, rows_per_slice, part);
  else if (D <= 32) gram_mfma_kernel<2><<<grid, block, 0, s>>>(x, N, D, rows_per_slice, part);
  else gram_mfma_kernel<4><<<grid, block, 0, s>>>(x, N, D, rows_per_slice, part);
}

void launch_canary(const int32_t* in, int32_t* out, int64_t n, int32_t offset, hipStream_t s) {
  canary_kernel<<<(unsigned)((n + 255) / 256), 256, 0, s>>>(in, out, n, offset);
}

}  // namespace gx
