// Full covariance at 16 < D <= 128: whitening E-step and weighted-Gram M-step
// on the bf16 MFMA with split operands (v_mfma_f32_32x32x16_bf16: every fp32
// operand as three bf16 parts, six bf16 products per fp32 product).
//
// The augmented formulation of em_tile.hip (features = the D(D+1)/2 products
// x_d x_e, split into bf16 parts) is built for D = 16; at larger D its feature
// rows outgrow the LDS.  Here the per-component quadratic form is formed as a
// squared norm instead, (x - μ)ᵀ Σ⁻¹ (x - μ) = ‖L⁻¹x - L⁻¹μ‖² with Σ = L Lᵀ
// (torch_fallback.py:400-432 computes the same value expanded, xᵀPx - 2xᵀPμ +
// μᵀPμ, clamped at zero; the norm is never negative and has no cancellation
// between the expanded terms), and the M-step statistics are the uncentered
// sums N_k = Σ r, Σ r·x and Σ r·x xᵀ the reference's matrix M-step reads
// (:3143-3167).
//
//   fw_pack_kernel   per component: the iteration prelude's weight, b = L⁻¹μ and
//                    the log2 constant in float64, and L⁻¹ split into three bf16
//                    parts (v = v1 + v2 + v3 exactly) laid out as the MFMA's A
//                    operand (one 16-deep chunk = 3 parts x 64 lanes x 8 values);
//   fw_estep_kernel  one wave per 32-row block, its rows split into three bf16
//                    parts as the B operand, every component in turn: the
//                    32 x 32 output tiles of y = L⁻¹x (rows i of L⁻¹ against the
//                    block's rows, k over x's columns; L⁻¹ is lower triangular, so
//                    tile t needs only the 16-deep chunks c <= 2t + 1), each
//                    product as the six bf16 MFMAs a1b3 + a3b1 + a2b2 + a1b2 +
//                    a2b1 + a1b1 (the dropped terms are below 2⁻²⁴ relative), one
//                    more MFMA adds -b from its three parts, and each lane sums the
//                    squares of its 16 entries; the partner lane (l ^ 32) holds the
//                    other 16.  The row's log-normaliser is accumulated online over
//                    the components; the log2 logits go to a (B, K, N) buffer;
//   fw_stats_kernel  one wave per component and row slice (D = 128:
//                    fw_stats128_kernel, two waves of five tiles each):
//                    Σ_n r_n x_n x_nᵀ = Σ w wᵀ with w = √r·x as the lower 32 x 32
//                    tiles over 16-row k-steps, one split of w serving as both
//                    operands; Σ r x and Σ r beside it on the VALU,
//                    r = 2^(l2 - lse2) from the E-step's buffers;
//   fw_proba_kernel  predict_proba: r = 2^(l2 - lse2) transposed to (B, N, K) (or
//                    the logits themselves, for the top-k selection).
//
// 32x32x16 bf16 MFMA operand layout: lane l supplies A[i = l % 32]
// [k = 8 (l / 32) .. +7] and B[k = 8 (l / 32) .. +7][j = l % 32]; accumulator
// register v of lane l holds C[8 (v / 4) + 4 (l / 32) + v % 4][l % 32].

#include <math.h>

#include <hip/hip_fp16.h>

#include "common.hpp"
#include "engine.hpp"

namespace gx {

namespace {

typedef float f32x16 __attribute__((ext_vector_type(16)));
typedef float f32x8 __attribute__((ext_vector_type(8)));
typedef __bf16 bf16x8v __attribute__((ext_vector_type(8)));
typedef __bf16 bf16x2 __attribute__((ext_vector_type(2)));

__device__ __forceinline__ f32x16 mfma32b(bf16x8v a, bf16x8v b, f32x16 c) {
  return __builtin_amdgcn_mfma_f32_32x32x16_bf16(a, b, c, 0, 0, 0);
}

// v = p1 + p2 + p3 exactly (three bf16 parts, each rounded to nearest even).
// The residuals v - p come from v_dot2_f32_bf16 against (-1, 0) / (0, -1), one
// instruction per value instead of a widening and a subtraction (the difference
// is exact, so the bits equal the subtract's for every finite input; a NaN or an
// infinity also turns its pair partner's lower parts into NaN).  The two
// constants pass through an empty asm so that they stay register operands: as
// an inline constant the compiler encodes (-1, 0) as the fp32 -1.0, whose bits
// the instruction reads as (0, -1).
__device__ __forceinline__ void split3v(f32x8 v, bf16x8v& p1, bf16x8v& p2, bf16x8v& p3) {
  uint32_t clo = 0x0000BF80u, chi = 0xBF800000u;
  asm("" : "+v"(clo), "+v"(chi));
  const bf16x2 nlo = __builtin_bit_cast(bf16x2, clo), nhi = __builtin_bit_cast(bf16x2, chi);
  p1 = __builtin_convertvector(v, bf16x8v);
  f32x8 r1, r2;
#pragma unroll
  for (int e = 0; e < 8; e += 2) {
    const bf16x2 q = bf16x2{p1[e], p1[e + 1]};
    r1[e] = __builtin_amdgcn_fdot2_f32_bf16(q, nlo, v[e], false);
    r1[e + 1] = __builtin_amdgcn_fdot2_f32_bf16(q, nhi, v[e + 1], false);
  }
  p2 = __builtin_convertvector(r1, bf16x8v);
#pragma unroll
  for (int e = 0; e < 8; e += 2) {
    const bf16x2 q = bf16x2{p2[e], p2[e + 1]};
    r2[e] = __builtin_amdgcn_fdot2_f32_bf16(q, nlo, r1[e], false);
    r2[e + 1] = __builtin_amdgcn_fdot2_f32_bf16(q, nhi, r1[e + 1], false);
  }
  p3 = __builtin_convertvector(r2, bf16x8v);
}

// Bytes of one 16-deep L⁻¹ chunk: three parts x 64 lanes x 8 bf16.
constexpr int kChunkBytes = 3 * 64 * 8 * 2;

// v of lane l % 32 plus v of lane l % 32 + 32, the same bits in both lanes
// (the swap yields the low half's value in one word and the high half's in the
// other, in every lane).
__device__ __forceinline__ float half_sum(float v) {
  const auto t = __builtin_amdgcn_permlane32_swap(__float_as_uint(v), __float_as_uint(v), false, false);
  return __uint_as_float(t[0]) + __uint_as_float(t[1]);
}

constexpr int kFwWaves = 4;

}  // namespace

// ---------------------------------------------------------------------------
// Operand packing (prelude, L⁻¹ chunks, -L⁻¹μ, constants)
// ---------------------------------------------------------------------------

__global__ __launch_bounds__(256) void fw_pack_kernel(FwPackArgs a) {
  __shared__ double red[4];
  __shared__ double bsh[128];
  const int k = blockIdx.x, b = blockIdx.y, t = threadIdx.x;
  const int K = a.K, D = a.D, DP = a.DP, NT = DP / 32, NCH = NT * (NT + 1);   // 16-deep chunks
  const size_t bk = (size_t)b * K + k;
  // Iteration prelude (torch_fallback.py:2061-2066): w <- max(w, min_weight) / Σ;
  // inference uses the weights as given.
  const float* wrow = a.weights + (size_t)b * K;
  float wk = wrow[k];
  if (a.prelude) {
    float sw = 0.f;
    for (int j = t; j < K; j += 256) sw += clamp_lo(wrow[j], a.min_weight);
    for (int off = 32; off >= 1; off /= 2) sw += __shfl_xor(sw, off);
    if ((t & 63) == 0) red[t >> 6] = (double)sw;
    __syncthreads();
    const float total = (float)red[0] + (float)red[1] + (float)red[2] + (float)red[3];
    wk = clamp_lo(wk, a.min_weight) / total;
    if (a.param_round == 1) wk = (float)(__bf16)wk;
    else if (a.param_round == 2) wk = (float)(__half)wk;
  }
  const float* X = a.linv + bk * D * D;
  const float* mu = a.means + bk * D;
  // b = L⁻¹μ in float64 (row i of L⁻¹ has entries j <= i)
  if (t < D) {
    double acc = 0.0;
    for (int j = 0; j <= t; ++j) acc = fma((double)X[t * D + j], (double)mu[j], acc);
    bsh[t] = acc;
  }
  __syncthreads();
  // -b as the A operand of one 32x32x16 MFMA against ones in k = 0..2: lane
  // l < 32 of tile tt holds the three parts of -b[32 tt + l] in k = 0..2.
  if (t < 64) {
    __bf16* aug = reinterpret_cast<__bf16*>(a.lpaug) + (bk * NT) * 512;
    for (int tt = 0; tt < NT; ++tt) {
      const int i = 32 * tt + (t & 31);
      const float v = (t < 32 && i < D) ? (float)(-bsh[i]) : 0.f;
      const __bf16 p1 = (__bf16)v;
      const float r1 = v - (float)p1;
      const __bf16 p2 = (__bf16)r1;
      const __bf16 p3 = (__bf16)(r1 - (float)p2);
      __bf16* dst = aug + (tt * 64 + t) * 8;
      dst[0] = p1;
      dst[1] = p2;
      dst[2] = p3;
      for (int e = 3; e < 8; ++e) dst[e] = (__bf16)0.f;
    }
  }
  if (t == 0) {
    constexpr double kLog2eD = 1.4426950408889634;
    const double c2 = (log((double)wk) - 0.5 * ((double)D * kLog2Pi + (double)a.logdet[bk])) * kLog2eD;
    a.cconst[bk] = make_float4((float)c2, 0.f, 0.f, 0.f);
  }
  // chunk j = (tile tt, 16-column chunk c <= 2 tt + 1), j = tt (tt + 1) + c;
  // part p, lane l, slot u: part p of L⁻¹[32 tt + l % 32][16 c + 8 (l / 32) + u]
  __bf16* lp = reinterpret_cast<__bf16*>(a.lpack) + bk * NCH * (kChunkBytes / 2);
  for (int e = t; e < NCH * 512; e += 256) {
    const int j = e >> 9, lane = (e >> 3) & 63, u = e & 7;
    int tt = 0;
    while ((tt + 1) * (tt + 2) <= j) ++tt;
    const int c = j - tt * (tt + 1);
    const int i = 32 * tt + (lane & 31), col = 16 * c + 8 * (lane >> 5) + u;
    const float v = (i < D && col < D) ? X[i * D + col] : 0.f;
    const __bf16 p1 = (__bf16)v;
    const float r1 = v - (float)p1;
    const __bf16 p2 = (__bf16)r1;
    __bf16* dst = lp + (size_t)j * (kChunkBytes / 2) + lane * 8 + u;
    dst[0] = p1;
    dst[512] = p2;
    dst[1024] = (__bf16)(r1 - (float)p2);
  }
}

// ---------------------------------------------------------------------------
// E-step: log2 logits, row log-normalisers, labels, log-likelihood partials
// ---------------------------------------------------------------------------

template <int DP>
__global__ __launch_bounds__(64 * kFwWaves) void fw_estep_kernel(FwArgs a) {
  constexpr int NT = DP / 32, NCH = NT * (NT + 1), XC = DP / 16;
  __shared__ double llw[kFwWaves];
  const int wave = threadIdx.x / 64, lane = threadIdx.x % 64, lr = lane & 31, h = lane >> 5;
  const int b = blockIdx.y;
  const int64_t N = a.N;
  const int D = a.D, K = a.K;
  const int64_t n0 = ((int64_t)blockIdx.x * kFwWaves + wave) * 32;
  const int64_t n = n0 + lr;
  const bool valid = n < N;

  // x block as the B operand in three bf16 parts: lane l holds row n, columns
  // 16 c + 8 h + u (u = 0..7) of 16-column chunk c.
  bf16x8v x1[XC], x2[XC], x3[XC];
  {
    const float* xrow = a.x + ((size_t)b * N + (valid ? n : 0)) * D;
#pragma unroll
    for (int c = 0; c < XC; ++c) {
      const int col0 = 16 * c + 8 * h;
      f32x8 v;
      if (a.vec_ok) {
        const f32x4 lo = valid ? *reinterpret_cast<const f32x4*>(xrow + col0) : f32x4{0.f, 0.f, 0.f, 0.f};
        const f32x4 hi = valid ? *reinterpret_cast<const f32x4*>(xrow + col0 + 4) : f32x4{0.f, 0.f, 0.f, 0.f};
        v = __builtin_shufflevector(lo, hi, 0, 1, 2, 3, 4, 5, 6, 7);
      } else {
#pragma unroll
        for (int u = 0; u < 8; ++u) v[u] = (valid && col0 + u < D) ? xrow[col0 + u] : 0.f;
      }
      split3v(v, x1[c], x2[c], x3[c]);
    }
  }
  // B operand of the -b step: ones in k = 0..2.
  bf16x8v ones;
#pragma unroll
  for (int u = 0; u < 8; ++u) ones[u] = (__bf16)((h == 0 && u < 3) ? 1.f : 0.f);

  // L⁻¹ chunks stream through a one-chunk prefetch; the buffer holds one spare
  // chunk after the last component, so the final prefetch stays in bounds.
  const char* lp = reinterpret_cast<const char*>(a.lpack) + (size_t)b * K * NCH * kChunkBytes + lane * 16;
  const bf16x8v* augp = reinterpret_cast<const bf16x8v*>(a.lpaug) + (size_t)b * K * NT * 64 + lane;
  bf16x8v nx[3];
#pragma unroll
  for (int p = 0; p < 3; ++p) nx[p] = *reinterpret_cast<const bf16x8v*>(lp + p * 1024);

  float m = -INFINITY, s = 0.f, best = -INFINITY;
  int bidx = 0;
  for (int k = 0; k < K; ++k) {
    const size_t bk = (size_t)b * K + k;
    bf16x8v augv[NT];
#pragma unroll
    for (int tt = 0; tt < NT; ++tt) augv[tt] = augp[((size_t)k * NT + tt) * 64];
    float q = 0.f;
#pragma unroll
    for (int tt = 0; tt < NT; ++tt) {
      // two accumulators, so consecutive MFMAs do not depend on each other; the
      // products of a chunk go smallest first
      f32x16 acc = mfma32b(augv[tt], ones, f32x16{}), acc2 = f32x16{};
#pragma unroll
      for (int c = 0; c <= 2 * tt + 1; ++c) {
        bf16x8v cur[3];
#pragma unroll
        for (int p = 0; p < 3; ++p) cur[p] = nx[p];
        lp += kChunkBytes;
#pragma unroll
        for (int p = 0; p < 3; ++p) nx[p] = *reinterpret_cast<const bf16x8v*>(lp + p * 1024);
        acc2 = mfma32b(cur[0], x3[c], acc2);
        acc = mfma32b(cur[2], x1[c], acc);
        acc2 = mfma32b(cur[1], x2[c], acc2);
        acc = mfma32b(cur[0], x2[c], acc);
        acc2 = mfma32b(cur[1], x1[c], acc2);
        acc = mfma32b(cur[0], x1[c], acc);
      }
#pragma unroll
      for (int v = 0; v < 16; ++v) {
        const float y = acc[v] + acc2[v];
        q = fmaf(y, y, q);
      }
    }
    q = half_sum(q);
    const float l2 = a.cconst[bk].x - 0.5f * kLog2e * q;
    if (l2 > m) {
      s = s * fast_exp2(m - l2) + 1.f;   // m = -inf: s is 0
      m = l2;
    } else if (l2 != -INFINITY) {
      s += fast_exp2(l2 - m);            // NaN passes through
    }
    if (l2 > best) {
      best = l2;
      bidx = k;
    }
    if (a.l2 && h == 0 && valid) a.l2[bk * N + n] = l2;
  }
  const float lse = a.hard ? best : m + __log2f(s);
  double ll = 0.0;
  if (h == 0 && valid) {
    a.lse2[(size_t)b * N + n] = lse;
    if (a.hard) a.hard_idx[(size_t)b * N + n] = bidx;
    if (a.scores) a.scores[(size_t)b * N + n] = lse * kLn2;
    if (a.labels) a.labels[(size_t)b * N + n] = bidx;
    ll = (double)lse * (double)kLn2;
  }
  if (a.ll_part) {
#pragma unroll
    for (int off = 32; off >= 1; off /= 2) ll += __shfl_xor(ll, off);
    if (lane == 0) llw[wave] = ll;
    __syncthreads();
    if (threadIdx.x == 0) {
      double sum = 0.0;
      for (int w = 0; w < kFwWaves; ++w) sum += llw[w];
      a.ll_part[(size_t)b * gridDim.x + blockIdx.x] = sum;
    }
  }
}

// ---------------------------------------------------------------------------
// M-step statistics: N_k, Σ r x, Σ r x xᵀ per component and row slice
// ---------------------------------------------------------------------------

template <int DP>
__global__ __launch_bounds__(64 * kFwWaves) void fw_stats_kernel(FwArgs a) {
  static_assert(DP <= 64, "D = 128 runs fw_stats128_kernel");
  constexpr int NT = DP / 32, NTT = NT * (NT + 1) / 2;
  const int wave = threadIdx.x / 64, lane = threadIdx.x % 64, lr = lane & 31, h = lane >> 5;
  const int b = blockIdx.z;
  const int k = blockIdx.y * kFwWaves + wave;
  if (k >= a.K) return;   // whole wave; the kernel has no barrier
  const int64_t N = a.N;
  const int D = a.D;
  const size_t bk = (size_t)b * a.K + k;
  const int64_t r0 = (int64_t)blockIdx.x * a.rows_per_slice;
  const int64_t r1 = (r0 + a.rows_per_slice < N) ? r0 + a.rows_per_slice : N;
  const float* xb = a.x + (size_t)b * N * D;
  const float* l2 = a.hard ? nullptr : a.l2 + bk * N;
  const float* lse2 = a.lse2 + (size_t)b * N;
  const int* hidx = a.hard ? a.hard_idx + (size_t)b * N : nullptr;
  const float* thr = a.thr2 ? a.thr2 + (size_t)b * N : nullptr;   // top-k mode
  const int* thri = a.thr2 ? a.thr_idx + (size_t)b * N : nullptr;

  f32x16 acc[NTT];
#pragma unroll
  for (int i = 0; i < NTT; ++i) acc[i] = f32x16{};
  float sx[NT];
#pragma unroll
  for (int c = 0; c < NT; ++c) sx[c] = 0.f;
  float sr = 0.f;

  for (int64_t n0 = r0; n0 < r1; n0 += 32) {
    const int64_t nr = n0 + lr;
    float rv = 0.f;
    if (nr < r1) {
      if (a.hard) {
        rv = hidx[nr] == k ? 1.f : 0.f;
      } else {
        const float l = l2[nr];
        const bool keep = !thr || l > thr[nr] || (l == thr[nr] && k <= thri[nr]);
        rv = keep ? fast_exp2(l - lse2[nr]) : 0.f;
      }
    }
    const float* xblk = xb + (size_t)n0 * D;           // the block's rows, 32-bit offsets below
    const int nrows = (int)((r1 - n0) < 32 ? (r1 - n0) : 32);
    // Split bf16 operands, 16 rows per k-step: lane (lr, h) holds rows 8h .. 8h+7
    // of the step at dims 32c + lr.  Σ r x xᵀ = Σ w wᵀ with w = √r·x, so one
    // three-way split of w is both the A and the B operand (Σ r x = Σ √r·w);
    // the six products of every lower tile go smallest first (consecutive
    // MFMAs into different tiles).  (The two steps stay a loop: unrolled, their
    // operands are live at once.)
#pragma unroll 1
    for (int s0 = 0; s0 < 32; s0 += 16) {
      f32x8 sq, xv[NT];
#pragma unroll
      for (int e = 0; e < 8; ++e) {
        const int src = s0 + 8 * h + e;
        const float r = __shfl(rv, src);
        sr += r;
        sq[e] = __builtin_amdgcn_sqrtf(r);
        const bool rowok = src < nrows;
#pragma unroll
        for (int c = 0; c < NT; ++c) {
          const int col = 32 * c + lr;
          xv[c][e] = (rowok && col < D) ? xblk[src * D + col] : 0.f;
        }
      }
      bf16x8v w1[NT], w2[NT], w3[NT];
#pragma unroll
      for (int c = 0; c < NT; ++c) {
        const f32x8 w = xv[c] * sq;
#pragma unroll
        for (int e = 0; e < 8; ++e) sx[c] = fmaf(sq[e], w[e], sx[c]);
        split3v(w, w1[c], w2[c], w3[c]);
      }
      auto products = [&](const bf16x8v (&pa)[NT], const bf16x8v (&pb)[NT]) {
        int ti = 0;
#pragma unroll
        for (int I = 0; I < NT; ++I)
#pragma unroll
          for (int J = 0; J <= I; ++J, ++ti) acc[ti] = mfma32b(pa[I], pb[J], acc[ti]);
      };
      products(w1, w3);
      products(w3, w1);
      products(w2, w2);
      products(w1, w2);
      products(w2, w1);
      products(w1, w1);
    }
  }

  // Statistics row: [Σ r x (DP) | Σ r x xᵀ packed (d <= e < DP, row by row) | N_k | 0 ...]
  float* out = a.part_stats + (((size_t)blockIdx.x * a.B + b) * a.K + k) * a.JP;
#pragma unroll
  for (int c = 0; c < NT; ++c) {
    const float tot = half_sum(sx[c]);
    if (h == 0) out[32 * c + lr] = tot;
  }
  int ti = 0;
#pragma unroll
  for (int I = 0; I < NT; ++I)
#pragma unroll
    for (int J = 0; J <= I; ++J, ++ti)
#pragma unroll
      for (int v = 0; v < 16; ++v) {
        const int gi = 32 * I + 8 * (v / 4) + 4 * h + (v % 4), gj = 32 * J + lr;
        if (gi >= gj) out[DP + fw_tri(DP, gj, gi)] = acc[ti][v];
      }
  const float nk = half_sum(sr);
  if (lane == 0) out[a.nk_col] = nk;
  if (lane >= 1 && a.nk_col + lane < a.JP) out[a.nk_col + lane] = 0.f;
}

// D = 128: two waves per component, each with five of the ten lower 32 x 32 tiles
// (tile rows {0, 3} and {1, 2}), so that the accumulators and the split operands
// of a wave fit two waves per SIMD; the same k-steps and operands as
// fw_stats_kernel's D <= 64 path.  Half 0 also forms Σ r x and N_k.
constexpr int kS128Tiles = 5;
constexpr int kS128I[2][kS128Tiles] = {{0, 3, 3, 3, 3}, {1, 1, 2, 2, 2}};
constexpr int kS128J[2][kS128Tiles] = {{0, 0, 1, 2, 3}, {0, 1, 0, 1, 2}};

template <int Q>
__device__ __forceinline__ void fw_stats128_half(const FwArgs& a, int k, int lane) {
  constexpr int DP = 128, NT = 4;
  constexpr int ND = Q == 0 ? 4 : 3;          // dims (32-wide) this half's tiles read
  const int lr = lane & 31, h = lane >> 5;
  const int b = blockIdx.z;
  const int64_t N = a.N;
  const int D = a.D;
  const size_t bk = (size_t)b * a.K + k;
  const int64_t r0 = (int64_t)blockIdx.x * a.rows_per_slice;
  const int64_t r1 = (r0 + a.rows_per_slice < N) ? r0 + a.rows_per_slice : N;
  const float* xb = a.x + (size_t)b * N * D;
  const float* l2 = a.hard ? nullptr : a.l2 + bk * N;
  const float* lse2 = a.lse2 + (size_t)b * N;
  const int* hidx = a.hard ? a.hard_idx + (size_t)b * N : nullptr;
  const float* thr = a.thr2 ? a.thr2 + (size_t)b * N : nullptr;   // top-k mode
  const int* thri = a.thr2 ? a.thr_idx + (size_t)b * N : nullptr;

  f32x16 acc[kS128Tiles];
#pragma unroll
  for (int i = 0; i < kS128Tiles; ++i) acc[i] = f32x16{};
  float sx[NT];
#pragma unroll
  for (int c = 0; c < NT; ++c) sx[c] = 0.f;
  float sr = 0.f;

  for (int64_t n0 = r0; n0 < r1; n0 += 32) {
    const int64_t nr = n0 + lr;
    float rv = 0.f;
    if (nr < r1) {
      if (a.hard) {
        rv = hidx[nr] == k ? 1.f : 0.f;
      } else {
        const float l = l2[nr];
        const bool keep = !thr || l > thr[nr] || (l == thr[nr] && k <= thri[nr]);
        rv = keep ? fast_exp2(l - lse2[nr]) : 0.f;
      }
    }
    const float* xblk = xb + (size_t)n0 * D;
    const int nrows = (int)((r1 - n0) < 32 ? (r1 - n0) : 32);
#pragma unroll 1
    for (int s0 = 0; s0 < 32; s0 += 16) {
      f32x8 sq, xv[ND];
#pragma unroll
      for (int e = 0; e < 8; ++e) {
        const int src = s0 + 8 * h + e;
        const float r = __shfl(rv, src);
        if (Q == 0) sr += r;
        sq[e] = __builtin_amdgcn_sqrtf(r);
        const bool rowok = src < nrows;
#pragma unroll
        for (int c = 0; c < ND; ++c) {
          const int col = 32 * c + lr;
          xv[c][e] = (rowok && col < D) ? xblk[src * D + col] : 0.f;
        }
      }
      bf16x8v w1[ND], w2[ND], w3[ND];
#pragma unroll
      for (int c = 0; c < ND; ++c) {
        const f32x8 w = xv[c] * sq;
        if (Q == 0) {
#pragma unroll
          for (int e = 0; e < 8; ++e) sx[c] = fmaf(sq[e], w[e], sx[c]);
        }
        split3v(w, w1[c], w2[c], w3[c]);
      }
      auto products = [&](const bf16x8v (&pa)[ND], const bf16x8v (&pb)[ND]) {
#pragma unroll
        for (int t = 0; t < kS128Tiles; ++t) acc[t] = mfma32b(pa[kS128I[Q][t]], pb[kS128J[Q][t]], acc[t]);
      };
      products(w1, w3);
      products(w3, w1);
      products(w2, w2);
      products(w1, w2);
      products(w2, w1);
      products(w1, w1);
    }
  }

  float* out = a.part_stats + (((size_t)blockIdx.x * a.B + b) * a.K + k) * a.JP;
  if (Q == 0) {
#pragma unroll
    for (int c = 0; c < NT; ++c) {
      const float tot = half_sum(sx[c]);
      if (h == 0) out[32 * c + lr] = tot;
    }
    const float nk = half_sum(sr);
    if (lane == 0) out[a.nk_col] = nk;
    if (lane >= 1 && a.nk_col + lane < a.JP) out[a.nk_col + lane] = 0.f;
  }
#pragma unroll
  for (int t = 0; t < kS128Tiles; ++t)
#pragma unroll
    for (int v = 0; v < 16; ++v) {
      const int gi = 32 * kS128I[Q][t] + 8 * (v / 4) + 4 * h + (v % 4), gj = 32 * kS128J[Q][t] + lr;
      if (gi >= gj) out[DP + fw_tri(DP, gj, gi)] = acc[t][v];
    }
}

__global__ __launch_bounds__(64 * kFwWaves) void fw_stats128_kernel(FwArgs a) {
  const int wave = threadIdx.x / 64, lane = threadIdx.x % 64;
  const int k = blockIdx.y * (kFwWaves / 2) + wave / 2;
  if (k >= a.K) return;   // whole wave; the kernel has no barrier
  if (wave % 2 == 0) fw_stats128_half<0>(a, k, lane);
  else fw_stats128_half<1>(a, k, lane);
}

// ---------------------------------------------------------------------------
// predict_proba: r[b][n][k] = 2^(l2[b][k][n] - lse2[b][n]), through a 32 x 32 LDS tile
// ---------------------------------------------------------------------------

__global__ __launch_bounds__(256) void fw_proba_kernel(const float* l2, const float* lse2, float* proba,
                                                       int64_t N, int K, bool raw) {
  __shared__ float tile[32][33];
  const int b = blockIdx.z;
  const int64_t n0 = (int64_t)blockIdx.x * 32;
  const int k0 = blockIdx.y * 32;
  const int tx = threadIdx.x & 31, ty = threadIdx.x >> 5;
  for (int kk = ty; kk < 32; kk += 8) {
    const int64_t n = n0 + tx;
    const int k = k0 + kk;
    float v = 0.f;
    if (n < N && k < K) {
      const float l = l2[((size_t)b * K + k) * N + n];
      v = raw ? l : fast_exp2(l - lse2[(size_t)b * N + n]);
    }
    tile[kk][tx] = v;
  }
  __syncthreads();
  for (int nn = ty; nn < 32; nn += 8) {
    const int64_t n = n0 + nn;
    const int k = k0 + tx;
    if (n < N && k < K) proba[((size_t)b * N + n) * K + k] = tile[tx][nn];
  }
}

// ---------------------------------------------------------------------------
// Launchers
// ---------------------------------------------------------------------------

int64_t fw_lpack_bytes(int B, int K, int DP) {
  const int NT = DP / 32;
  return ((int64_t)B * K * (NT * (NT + 1)) + 1) * kChunkBytes;
}

int fw_eblocks(int64_t N) { return (int)((N + 32 * kFwWaves - 1) / (32 * kFwWaves)); }

void launch_fw_pack(const FwPackArgs& a, hipStream_t s) {
  fw_pack_kernel<<<dim3(a.K, a.B), 256, 0, s>>>(a);
}

template <int DP>
static void launch_fw_dp(int phase, const FwArgs& a, int slices, hipStream_t s) {
  if (phase == 0)
    fw_estep_kernel<DP><<<dim3(fw_eblocks(a.N), a.B), 64 * kFwWaves, 0, s>>>(a);
  else if constexpr (DP == 128)
    fw_stats128_kernel<<<dim3(slices, (a.K + kFwWaves / 2 - 1) / (kFwWaves / 2), a.B), 64 * kFwWaves, 0, s>>>(a);
  else
    fw_stats_kernel<DP><<<dim3(slices, (a.K + kFwWaves - 1) / kFwWaves, a.B), 64 * kFwWaves, 0, s>>>(a);
}

int launch_fw(int dp, int phase, const FwArgs& a, int slices, hipStream_t s) {
  switch (dp) {
    case 32: launch_fw_dp<32>(phase, a, slices, s); return 0;
    case 64: launch_fw_dp<64>(phase, a, slices, s); return 0;
    case 128: launch_fw_dp<128>(phase, a, slices, s); return 0;
    default: return -1;
  }
}

void launch_fw_proba(const float* l2, const float* lse2, float* proba, int B, int64_t N, int K, hipStream_t s,
                     bool raw) {
  fw_proba_kernel<<<dim3((unsigned)((N + 31) / 32), (K + 31) / 32, B), 256, 0, s>>>(l2, lse2, proba, N, K, raw);
}

}  // namespace gx
