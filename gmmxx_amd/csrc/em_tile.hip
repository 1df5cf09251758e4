// The GMM EM tile kernel for gfx950 (CDNA4).
//
// One workgroup owns a tile of KT = nwaves * CW mixture components and a
// contiguous slice of rows of one batch.  Each wave keeps the E-step operand W
// for its CW components resident in VGPRs as MFMA fragments for the whole
// launch.  Per block of 32 rows the workgroup stages x into LDS, builds the
// augmented row features, and then:
//
//   MODE_LSE    E-GEMM in "component rows" orientation (C = W·φᵀ) so a lane
//               holds several components of one data row; per-row max,
//               scaled sum and first-index argmax over the tile are reduced
//               across lanes (2 shuffles) and waves (LDS) and written as a
//               per-k-tile partial.
//   MODE_STATS  E-GEMM in "data rows" orientation (C = φ·Wᵀ); the epilogue turns
//               logits into responsibilities r = 2^(l2 - lse2) in registers and
//               feeds them directly as the A operand of the M-GEMM
//               acc += rᵀ·ψ, so the (B, N, K) responsibility matrix never
//               exists.  Each workgroup writes one partial statistics tile.
//   MODE_PROBA  Same epilogue; r is written out (predict_proba needs it).
//
// Logits are kept in log2 units (l2 = l·log2 e) so exp2 maps to v_exp_f32.
// bf16 inputs multiply exact bf16 x against a hi/lo bf16 split of the fp32
// operand, which keeps the cross term at fp32-oracle noise level.

#include <type_traits>

#include "common.hpp"
#include "engine.hpp"

namespace gx {

template <int COV, int DP, bool BF>
__host__ __device__ constexpr int cw_for() {
  return (COV == FULL) ? 16 : ((COV == DIAG && DP >= 128) ? 16 : 32);
}

template <typename T>
__device__ __forceinline__ T ld16(const void* p) { return *reinterpret_cast<const T*>(p); }

template <int COV, typename XT, int DP, int CW, int MODE>
__global__ __launch_bounds__(512) void em_tile_kernel(TileArgs a) {
  constexpr bool BF = sizeof(XT) == 2;
  using Dm = Dims<COV, DP, BF>;
  constexpr int EP = Dm::EP, JP = Dm::JP, J = Dm::J, S = Dm::S;
  constexpr int CT = CW / 16;
  constexpr int ECH = BF ? EP / 32 : EP / 16;
  constexpr int JT = JP / 16;
  constexpr int XS = DP + (BF ? 8 : 4);                 // xs row stride, elements
  constexpr int PS = EP + 4;                             // φ row stride (full only)
  constexpr int QS = kBN + (BF ? 8 : 4);                 // ψᵀ row stride, elements
  constexpr float SC = (COV == SPH || COV == TIED) ? -2.f : 1.f;
  using FT = typename std::conditional<BF, __bf16, float>::type;
  using WF = typename std::conditional<BF, bf16x8, f32x4>::type;

  __shared__ __align__(16) XT xs[kBN * XS];
  __shared__ __align__(16) float phi[COV == FULL ? kBN * PS : 4];
  __shared__ __align__(16) FT psiT[MODE == MODE_STATS ? JP * QS : 8];
  __shared__ float rowq_s[kBN];
  __shared__ float lse_s[kBN];
  __shared__ float red_m[MODE == MODE_LSE ? 8 * kBN : 1];
  __shared__ float red_s[MODE == MODE_LSE ? 8 * kBN : 1];
  __shared__ int red_i[MODE == MODE_LSE ? 8 * kBN : 1];

  const int tid = threadIdx.x;
  const int nthr = blockDim.x;
  const int nw = nthr / 64;
  const int wave = tid / 64, lane = tid % 64;
  const int g = lane / 16, li = lane % 16;
  const int b = blockIdx.y;
  const int64_t N = a.N;
  const int K = a.K, D = a.D;

  // XCD-aware block mapping: consecutive logical ids land on one XCD, so the
  // k-tiles that share a row slice are co-scheduled and hit the same L2.
  const int G = gridDim.x, id = blockIdx.x;
  const int L = (G % 8 == 0) ? (id % 8) * (G / 8) + id / 8 : id;
  const int ktile = L % a.ktiles, slice = L / a.ktiles;
  const int kbase = ktile * nw * CW + wave * CW;
  const int64_t rbeg = (int64_t)slice * a.rows_per_slice;
  const int64_t rend = (rbeg + a.rows_per_slice < N) ? rbeg + a.rows_per_slice : N;

  // ---- resident E-step operand and per-component constants ----
  WF whi[CT][ECH];
  WF wlo[BF ? CT : 1][BF ? ECH : 1];
#pragma unroll
  for (int ct = 0; ct < CT; ++ct) {
    const int kk = kbase + 16 * ct + li;
#pragma unroll
    for (int ec = 0; ec < ECH; ++ec) {
      const int e0 = BF ? 32 * ec + 8 * g : 16 * ec + 4 * g;
      if (kk < K) {
        const size_t off = ((size_t)b * K + kk) * EP + e0;
        if constexpr (BF) {
          whi[ct][ec] = ld16<bf16x8>(reinterpret_cast<const __bf16*>(a.w_hi) + off);
          wlo[ct][ec] = ld16<bf16x8>(reinterpret_cast<const __bf16*>(a.w_lo) + off);
        } else {
          whi[ct][ec] = ld16<f32x4>(reinterpret_cast<const float*>(a.w_hi) + off);
        }
      } else {
        if constexpr (BF) {
#pragma unroll
          for (int s = 0; s < 8; ++s) { whi[ct][ec][s] = (__bf16)0.f; wlo[ct][ec][s] = (__bf16)0.f; }
        } else {
          whi[ct][ec] = f32x4{0.f, 0.f, 0.f, 0.f};
        }
      }
    }
  }
  const float4 kInvalid = make_float4(0.f, 0.f, -INFINITY, 0.f);
  float4 cS[CT];           // data-row orientation: component kbase + 16ct + li
  float4 cL[CT][4];        // component-row orientation: kbase + 16ct + 4g + v
#pragma unroll
  for (int ct = 0; ct < CT; ++ct) {
    const int k1 = kbase + 16 * ct + li;
    cS[ct] = (k1 < K) ? a.cconst[(size_t)b * K + k1] : kInvalid;
#pragma unroll
    for (int v = 0; v < 4; ++v) {
      const int k2 = kbase + 16 * ct + 4 * g + v;
      cL[ct][v] = (k2 < K) ? a.cconst[(size_t)b * K + k2] : kInvalid;
    }
  }

  f32x4 acc[MODE == MODE_STATS ? CT : 1][MODE == MODE_STATS ? JT : 1];
  if constexpr (MODE == MODE_STATS) {
#pragma unroll
    for (int ct = 0; ct < CT; ++ct)
#pragma unroll
      for (int jt = 0; jt < JT; ++jt) acc[ct][jt] = f32x4{0.f, 0.f, 0.f, 0.f};
    // ψᵀ padding rows [J, JP) stay zero for the whole launch.
    for (int i = tid; i < (JP - J) * QS; i += nthr) psiT[J * QS + i] = (FT)0.f;
  }

  const XT* xb = reinterpret_cast<const XT*>(a.x) + (size_t)b * N * D;

  // φ fragment (4 consecutive E-step features of one LDS row), fp32 path.
  auto phi4 = [&](int r, int e0) -> f32x4 {
    if constexpr (COV == FULL) {
      return ld16<f32x4>(&phi[r * PS + e0]);
    } else if constexpr (COV == DIAG) {
      const int c = e0 < DP ? e0 : e0 - DP;
      f32x4 v = ld16<f32x4>(&xs[r * XS + c]);
      if (e0 < DP) v = v * v;
      return v;
    } else {
      return ld16<f32x4>(&xs[r * XS + e0]);
    }
  };

  for (int64_t n0 = rbeg; n0 < rend; n0 += kBN) {
    __syncthreads();
    // ---- stage x rows [n0, n0 + 32) into LDS, zero-padded ----
    constexpr int VEC = 16 / sizeof(XT);
    if (a.vec_ok) {
      for (int c = tid; c < kBN * DP / VEC; c += nthr) {
        const int r = c / (DP / VEC), cc = (c % (DP / VEC)) * VEC;
        const int64_t n = n0 + r;
        if (n < rend) {
          *reinterpret_cast<uint4*>(&xs[r * XS + cc]) =
              *reinterpret_cast<const uint4*>(xb + (size_t)n * D + cc);
        } else {
          *reinterpret_cast<uint4*>(&xs[r * XS + cc]) = make_uint4(0, 0, 0, 0);
        }
      }
    } else {
      for (int c = tid; c < kBN * DP; c += nthr) {
        const int r = c / DP, cc = c % DP;
        const int64_t n = n0 + r;
        xs[r * XS + cc] = (n < rend && cc < D) ? xb[(size_t)n * D + cc] : (XT)0.f;
      }
    }
    __syncthreads();

    // ---- row quantities and feature tiles ----
    if (tid < kBN) {
      const int r = tid;
      const int64_t n = n0 + r;
      float q = 0.f;
      if constexpr (COV == SPH) {
        for (int d = 0; d < DP; ++d) { const float v = to_f32(xs[r * XS + d]); q = fmaf(v, v, q); }
      } else if constexpr (COV == TIED) {
        q = (n < rend) ? a.rowq[(size_t)b * N + n] : 0.f;
      }
      rowq_s[r] = q;
      if constexpr (MODE != MODE_LSE) lse_s[r] = (n < rend) ? a.lse2[(size_t)b * N + n] : INFINITY;
      if constexpr (MODE == MODE_STATS && COV == SPH) {
        if constexpr (BF) {
          const __bf16 hi = (__bf16)q;
          psiT[(DP + 1) * QS + r] = hi;
          psiT[(DP + 2) * QS + r] = (__bf16)(q - (float)hi);
        } else {
          psiT[(DP + 1) * QS + r] = q;
          psiT[(DP + 2) * QS + r] = 0.f;
        }
        psiT[DP * QS + r] = (FT)1.f;
      }
    }
    if constexpr (MODE == MODE_STATS) {
      for (int i = tid; i < DP * kBN; i += nthr) {
        const int d = i / kBN, r = i % kBN;
        const XT v = xs[r * XS + d];
        psiT[d * QS + r] = (FT)v;
        if constexpr (COV == DIAG) { const float f = to_f32(v); psiT[(DP + d) * QS + r] = f * f; }
      }
      if constexpr (COV == DIAG || COV == TIED) {
        for (int r = tid; r < kBN; r += nthr) psiT[(COV == DIAG ? 2 * DP : DP) * QS + r] = (FT)1.f;
      }
    }
    if constexpr (COV == FULL) {
      for (int i = tid; i < kBN * DP; i += nthr) {
        const int r = i / DP, d = i % DP;
        const float xd = to_f32(xs[r * XS + d]);
        for (int e = d; e < DP; ++e) {
          const float p = xd * to_f32(xs[r * XS + e]);
          const int s = sym_index(d, e, DP);
          phi[r * PS + s] = p;
          if constexpr (MODE == MODE_STATS) psiT[(DP + s) * QS + r] = p;
        }
        phi[r * PS + S + d] = xd;
      }
      for (int i = tid; i < kBN * (EP - S - DP); i += nthr) {
        const int r = i / (EP - S - DP), c = i % (EP - S - DP);
        phi[r * PS + S + DP + c] = 0.f;
      }
      if constexpr (MODE == MODE_STATS)
        for (int r = tid; r < kBN; r += nthr) psiT[(DP + S) * QS + r] = 1.f;
    }
    __syncthreads();

    if constexpr (MODE == MODE_LSE) {
      // ---- E-GEMM, component-row orientation: T[ct][nt] = W(16 comps) · φᵀ(16 rows) ----
      f32x4 T[CT][2];
#pragma unroll
      for (int ct = 0; ct < CT; ++ct) { T[ct][0] = f32x4{0.f, 0.f, 0.f, 0.f}; T[ct][1] = T[ct][0]; }
#pragma unroll
      for (int ec = 0; ec < ECH; ++ec) {
        if constexpr (BF) {
          bf16x8 bx[2];
#pragma unroll
          for (int nt = 0; nt < 2; ++nt) bx[nt] = ld16<bf16x8>(&xs[(16 * nt + li) * XS + 32 * ec + 8 * g]);
#pragma unroll
          for (int ct = 0; ct < CT; ++ct)
#pragma unroll
            for (int nt = 0; nt < 2; ++nt) {
              T[ct][nt] = mfma_bf16(whi[ct][ec], bx[nt], T[ct][nt]);
              T[ct][nt] = mfma_bf16(wlo[ct][ec], bx[nt], T[ct][nt]);
            }
        } else {
          f32x4 b4[2];
#pragma unroll
          for (int nt = 0; nt < 2; ++nt) b4[nt] = phi4(16 * nt + li, 16 * ec + 4 * g);
#pragma unroll
          for (int ct = 0; ct < CT; ++ct)
#pragma unroll
            for (int nt = 0; nt < 2; ++nt)
#pragma unroll
              for (int t = 0; t < 4; ++t) T[ct][nt] = mfma_f32(whi[ct][ec][t], b4[nt][t], T[ct][nt]);
        }
      }
      // ---- per data row: max / argmax / scaled sum over this wave's components ----
#pragma unroll
      for (int nt = 0; nt < 2; ++nt) {
        const int r = 16 * nt + li;
        const float rq = rowq_s[r];
        float l2v[CT][4];
        float m = -INFINITY;
        int idx = 0x7fffffff;
#pragma unroll
        for (int ct = 0; ct < CT; ++ct)
#pragma unroll
          for (int v = 0; v < 4; ++v) {
            float t = fmaf(T[ct][nt][v], SC, rq + cL[ct][v].x);
            t = fmaxf(t, 0.f);
            const float l2 = fmaf(t, cL[ct][v].y, cL[ct][v].z);
            l2v[ct][v] = l2;
            if (l2 > m) { m = l2; idx = kbase + 16 * ct + 4 * g + v; }
          }
        float s = 0.f;
        if (m != -INFINITY) {
#pragma unroll
          for (int ct = 0; ct < CT; ++ct)
#pragma unroll
            for (int v = 0; v < 4; ++v) s += fast_exp2(l2v[ct][v] - m);
        }
#pragma unroll
        for (int off = 16; off <= 32; off *= 2) {
          const float m2 = __shfl_xor(m, off);
          const float s2 = __shfl_xor(s, off);
          const int i2 = __shfl_xor(idx, off);
          lse_merge(m, s, idx, m2, s2, i2);
        }
        if (g == 0) {
          red_m[wave * kBN + r] = m;
          red_s[wave * kBN + r] = s;
          red_i[wave * kBN + r] = idx;
        }
      }
      __syncthreads();
      if (tid < kBN) {
        const int64_t n = n0 + tid;
        float m = red_m[tid], s = red_s[tid];
        int idx = red_i[tid];
        for (int w = 1; w < nw; ++w) lse_merge(m, s, idx, red_m[w * kBN + tid], red_s[w * kBN + tid], red_i[w * kBN + tid]);
        if (n < rend) {
          const size_t o = ((size_t)ktile * a.B + b) * N + n;
          a.part_ms[2 * o] = m;
          a.part_ms[2 * o + 1] = s;
          a.part_idx[o] = idx;
        }
      }
    } else {
      // ---- E-GEMM, data-row orientation: S[rt][ct] = φ(16 rows) · Wᵀ(16 comps) ----
      f32x4 Sv[2][CT];
#pragma unroll
      for (int ct = 0; ct < CT; ++ct) { Sv[0][ct] = f32x4{0.f, 0.f, 0.f, 0.f}; Sv[1][ct] = Sv[0][ct]; }
#pragma unroll
      for (int ec = 0; ec < ECH; ++ec) {
        if constexpr (BF) {
          // Row permutation: tile rt, A-row i  ->  data row 8(i/4) + 4rt + i%4, so that
          // C-row 4g+v of tile rt is data row 8g + 4rt + v (8 consecutive rows per lane group).
          bf16x8 ax[2];
#pragma unroll
          for (int rt = 0; rt < 2; ++rt) ax[rt] = ld16<bf16x8>(&xs[(8 * (li / 4) + 4 * rt + (li % 4)) * XS + 32 * ec + 8 * g]);
#pragma unroll
          for (int ct = 0; ct < CT; ++ct)
#pragma unroll
            for (int rt = 0; rt < 2; ++rt) {
              Sv[rt][ct] = mfma_bf16(ax[rt], whi[ct][ec], Sv[rt][ct]);
              Sv[rt][ct] = mfma_bf16(ax[rt], wlo[ct][ec], Sv[rt][ct]);
            }
        } else {
          f32x4 a4[2];
#pragma unroll
          for (int rt = 0; rt < 2; ++rt) a4[rt] = phi4(16 * rt + li, 16 * ec + 4 * g);
#pragma unroll
          for (int ct = 0; ct < CT; ++ct)
#pragma unroll
            for (int rt = 0; rt < 2; ++rt)
#pragma unroll
              for (int t = 0; t < 4; ++t) Sv[rt][ct] = mfma_f32(a4[rt][t], whi[ct][ec][t], Sv[rt][ct]);
        }
      }
#pragma unroll
      for (int ct = 0; ct < CT; ++ct) {
        const float4 c = cS[ct];
        float rr[2][4];
#pragma unroll
        for (int rt = 0; rt < 2; ++rt)
#pragma unroll
          for (int v = 0; v < 4; ++v) {
            const int r = BF ? 8 * g + 4 * rt + v : 16 * rt + 4 * g + v;
            float t = fmaf(Sv[rt][ct][v], SC, rowq_s[r] + c.x);
            t = fmaxf(t, 0.f);
            const float l2 = fmaf(t, c.y, c.z);
            rr[rt][v] = fast_exp2(l2 - lse_s[r]);
          }
        if constexpr (MODE == MODE_STATS) {
          if constexpr (BF) {
            bf16x8 ar;
#pragma unroll
            for (int rt = 0; rt < 2; ++rt)
#pragma unroll
              for (int v = 0; v < 4; ++v) ar[4 * rt + v] = (__bf16)rr[rt][v];
#pragma unroll
            for (int jt = 0; jt < JT; ++jt) {
              const bf16x8 bq = ld16<bf16x8>(&psiT[(16 * jt + li) * QS + 8 * g]);
              acc[ct][jt] = mfma_bf16(ar, bq, acc[ct][jt]);
            }
          } else {
#pragma unroll
            for (int jt = 0; jt < JT; ++jt)
#pragma unroll
              for (int rt = 0; rt < 2; ++rt) {
                const f32x4 bq = ld16<f32x4>(&psiT[(16 * jt + li) * QS + 16 * rt + 4 * g]);
#pragma unroll
                for (int v = 0; v < 4; ++v) acc[ct][jt] = mfma_f32(rr[rt][v], bq[v], acc[ct][jt]);
              }
          }
        } else {  // MODE_PROBA
          const int kk = kbase + 16 * ct + li;
          if (kk < K) {
#pragma unroll
            for (int rt = 0; rt < 2; ++rt)
#pragma unroll
              for (int v = 0; v < 4; ++v) {
                const int r = BF ? 8 * g + 4 * rt + v : 16 * rt + 4 * g + v;
                const int64_t n = n0 + r;
                if (n < rend) a.proba[((size_t)b * N + n) * K + kk] = rr[rt][v];
              }
          }
        }
      }
    }
  }

  if constexpr (MODE == MODE_STATS) {
#pragma unroll
    for (int ct = 0; ct < CT; ++ct)
#pragma unroll
      for (int v = 0; v < 4; ++v) {
        const int kk = kbase + 16 * ct + 4 * g + v;
        if (kk < K) {
          float* dst = a.part_stats + (((size_t)slice * a.B + b) * K + kk) * JP;
#pragma unroll
          for (int jt = 0; jt < JT; ++jt) dst[16 * jt + li] = acc[ct][jt][v];
        }
      }
  }
}

template <int COV, typename XT, int DP>
static int launch_tile_t(int mode, const TileArgs& a, dim3 grid, int nw, hipStream_t s) {
  constexpr int CW = cw_for<COV, DP, sizeof(XT) == 2>();
  const dim3 block(64 * nw);
  switch (mode) {
    case MODE_LSE: em_tile_kernel<COV, XT, DP, CW, MODE_LSE><<<grid, block, 0, s>>>(a); break;
    case MODE_STATS: em_tile_kernel<COV, XT, DP, CW, MODE_STATS><<<grid, block, 0, s>>>(a); break;
    case MODE_PROBA: em_tile_kernel<COV, XT, DP, CW, MODE_PROBA><<<grid, block, 0, s>>>(a); break;
    default: return -1;
  }
  return 0;
}

int tile_cw(int cov, int dp, int bf) {
  if (cov == FULL) return 16;
  if (cov == DIAG && dp >= 128) return 16;
  (void)bf;
  return 32;
}

template <int COV, typename XT>
static int launch_tile_dp(int dp, int mode, const TileArgs& a, dim3 grid, int nw, hipStream_t s) {
  switch (dp) {
    case 16: return launch_tile_t<COV, XT, 16>(mode, a, grid, nw, s);
    case 32: return launch_tile_t<COV, XT, 32>(mode, a, grid, nw, s);
    case 64: return launch_tile_t<COV, XT, 64>(mode, a, grid, nw, s);
    case 128: return launch_tile_t<COV, XT, 128>(mode, a, grid, nw, s);
    default: return -1;
  }
}

int launch_tile(int cov, int bf, int dp, int mode, const TileArgs& a, dim3 grid, int nw, hipStream_t s) {
  switch (cov) {
    case SPH:
      return bf ? launch_tile_dp<SPH, __bf16>(dp, mode, a, grid, nw, s)
                : launch_tile_dp<SPH, float>(dp, mode, a, grid, nw, s);
    case DIAG:
      return bf ? -1 : launch_tile_dp<DIAG, float>(dp, mode, a, grid, nw, s);
    case TIED:
      return bf ? -1 : launch_tile_dp<TIED, float>(dp, mode, a, grid, nw, s);
    case FULL:
      return (bf || dp != 16) ? -1 : launch_tile_t<FULL, float, 16>(mode, a, grid, nw, s);
    default:
      return -1;
  }
}

}  // namespace gx
