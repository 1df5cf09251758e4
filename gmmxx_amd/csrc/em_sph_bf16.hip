// Spherical-covariance tile kernel for bf16 x (the large-K, D <= 128 hot path).
//
// Same two-pass structure and launch geometry as the generic tile kernel
// (em_tile.hip), with the per-element affine work moved into the MFMA:
//
//   l2(n, k) = A_k·‖x_n‖² + x_n·W'_k + C_k        (log2 units)
//   W'_k = log2(e)·μ_k / σ²_k                       (bf16 hi + lo split)
//
// Every staged row carries a 32-column augmented chunk next to x and every
// component a matching 32-column chunk of constants, so one extra MFMA per
// 16x16 output tile produces the full logit:
//
//   row side  [q_h q_m q_l q_h q_m q_h 1 1 | 1 0 ...]
//   comp side [A_h A_h A_h A_m A_m A_l C_h C_m | C_l 0 ...]
//
// with q = ‖x‖² and _h/_m/_l the three-way bf16 split of an fp32 value
// (v = h + m + l to ~2^-24 relative).  The dropped cross products (A_m·q_l,
// A_l·q_m, A_l·q_l) are below 2^-31 of A·q.  Both passes compute the logit
// with the same MFMA chain, so the statistics pass reproduces the
// log-normaliser pass's logits bit for bit and responsibilities sum to 1.
// The epilogues are then
//   log-normaliser pass: row max (max3 + lane swaps), exp2(l2 - max), sum;
//   statistics pass:     r = exp2(l2 - lse2), packed to bf16 as the A operand
//                        of the M-GEMM acc_stats += rᵀ·ψ (ψ = [x | 1 | q_h | q_l]).
// Padding components carry C = -1e30 and padding rows lse2 = +1e30, so their
// exponentials are exactly 0 without infinities inside the MFMA.

#include "common.hpp"
#include "engine.hpp"

namespace gx {

namespace {

constexpr int kAug = 32;         // augmented k-chunk width (bf16 columns)
constexpr float kHuge = 1e30f;   // "minus infinity" that stays finite through MFMA

template <typename T>
__device__ __forceinline__ T ld16(const void* p) { return *reinterpret_cast<const T*>(p); }

template <int CTRL>
__device__ __forceinline__ float dpp(float v) {
  return __int_as_float(__builtin_amdgcn_update_dpp(0, __float_as_int(v), CTRL, 0xF, 0xF, false));
}

// Sum / max / min over groups of G consecutive lanes (G <= 16), result in every lane.
template <int G>
__device__ __forceinline__ float group_sum(float v) {
  if constexpr (G >= 2) v += dpp<0xB1>(v);    // lane ^ 1
  if constexpr (G >= 4) v += dpp<0x4E>(v);    // lane ^ 2
  if constexpr (G >= 8) v += dpp<0x141>(v);   // row_half_mirror
  if constexpr (G >= 16) v += dpp<0x140>(v);  // row_mirror
  return v;
}
template <int G>
__device__ __forceinline__ float group_max(float v) {
  if constexpr (G >= 2) v = fmaxf(v, dpp<0xB1>(v));
  if constexpr (G >= 4) v = fmaxf(v, dpp<0x4E>(v));
  if constexpr (G >= 8) v = fmaxf(v, dpp<0x141>(v));
  if constexpr (G >= 16) v = fmaxf(v, dpp<0x140>(v));
  return v;
}
template <int G>
__device__ __forceinline__ int group_min_i(int v) {
  if constexpr (G >= 2) v = min(v, __builtin_amdgcn_update_dpp(0, v, 0xB1, 0xF, 0xF, false));
  if constexpr (G >= 4) v = min(v, __builtin_amdgcn_update_dpp(0, v, 0x4E, 0xF, 0xF, false));
  if constexpr (G >= 8) v = min(v, __builtin_amdgcn_update_dpp(0, v, 0x141, 0xF, 0xF, false));
  if constexpr (G >= 16) v = min(v, __builtin_amdgcn_update_dpp(0, v, 0x140, 0xF, 0xF, false));
  return v;
}

// v combined with lane l ^ 16 (OFF = 16) or l ^ 32 (OFF = 32).
template <int OFF, bool MAX>
__device__ __forceinline__ float lanes_op(float v) {
  const auto t = (OFF == 16) ? __builtin_amdgcn_permlane16_swap(__float_as_uint(v), __float_as_uint(v), false, false)
                             : __builtin_amdgcn_permlane32_swap(__float_as_uint(v), __float_as_uint(v), false, false);
  const float a = __uint_as_float(t[0]), b = __uint_as_float(t[1]);
  return MAX ? fmaxf(a, b) : a + b;
}
template <int OFF>
__device__ __forceinline__ int lanes_min_i(int v) {
  const auto t = (OFF == 16) ? __builtin_amdgcn_permlane16_swap((unsigned)v, (unsigned)v, false, false)
                             : __builtin_amdgcn_permlane32_swap((unsigned)v, (unsigned)v, false, false);
  return min((int)t[0], (int)t[1]);
}

__device__ __forceinline__ void split3(float v, __bf16& h, __bf16& m, __bf16& l) {
  h = (__bf16)v;
  const float r = v - (float)h;
  m = (__bf16)r;
  l = (__bf16)(r - (float)m);
}

__device__ __forceinline__ uint32_t pack2(__bf16 a, __bf16 b) {
  return (uint32_t)__builtin_bit_cast(uint16_t, a) | ((uint32_t)__builtin_bit_cast(uint16_t, b) << 16);
}

}  // namespace

template <int DP, int NW, int MODE>
__global__ __launch_bounds__(64 * NW) void sph_bf16_kernel(TileArgs a) {
  constexpr bool LSE = (MODE == MODE_LSE || MODE == MODE_LSE_IDX);
  constexpr bool WANT_IDX = MODE == MODE_LSE_IDX;
  constexpr bool STATS = MODE == MODE_STATS || MODE == MODE_STATS_TOPK;
  constexpr bool TOPK = MODE == MODE_STATS_TOPK;
  constexpr int CW = 32, CT = 2;                 // components per wave, 16-wide tiles
  constexpr int ECH = DP / 32;                   // x chunks of the E-GEMM
  // Staged row stride (bf16): s = XS/2 dwords ≡ 8 or 24 (mod 32) measured fastest for
  // both the b128 E-GEMM reads (16 consecutive rows, one column) and the
  // transposing ψ reads (4 rows x 32 bytes); s = 40, 56, 88.
  constexpr int XS = DP <= 32 ? 80 : (DP <= 64 ? 112 : 176);
  static_assert(DP + kAug <= XS, "row does not fit the staging stride");
  constexpr int JT = DP / 16 + 1;                // ψ = the staged row: [x | augmented columns 0..15]
  constexpr int JP = 16 * JT;                    // statistics row length
  // Wide rows: the statistics/proba passes read the augmented chunk the
  // log-normaliser pass stored (16 bytes per row) instead of recomputing ‖x‖²;
  // narrow rows are HBM bound, where the extra bytes cost more than the VALU.
  constexpr bool AUX = DP >= 128;
  constexpr int CPR = DP / 8;                    // 16-byte chunks per row
  constexpr int NCH = kBN * CPR;                 // chunks per row block
  constexpr int NTHR = 64 * NW;
  constexpr int PF = (NCH + NTHR - 1) / NTHR;    // chunks per thread
  constexpr int NB = 3;                          // staged-row buffers (loader runs 2 blocks ahead)
  static_assert(NCH % 64 == 0, "row block must split into whole waves of chunks");

  __shared__ __align__(16) __bf16 xs[NB * kBN * XS];
  __shared__ __align__(16) float lse_s[LSE ? 4 : NB * kBN];
  __shared__ __align__(16) float thr_s[TOPK ? NB * kBN : 4];   // top-k threshold logit and index per row
  __shared__ __align__(16) int thri_s[TOPK ? NB * kBN : 4];
  constexpr int RS = kBN + 1;                    // red_* stride per wave (conflict-free reads)
  __shared__ float red_m[LSE ? 2 * NW * RS : 1];   // [parity][wave][row]
  __shared__ float red_s[LSE ? 2 * NW * RS : 1];
  __shared__ int red_i[WANT_IDX ? 2 * NW * RS : 1];

  const int tid = threadIdx.x;
  const int wave = tid / 64, lane = tid % 64;
  const int g = lane / 16, li = lane % 16;
  const int b = blockIdx.y;
  const int64_t N = a.N;
  const int K = a.K, D = a.D;

  // XCD-aware block mapping (component tiles of one row slice share an L2).
  const int G = gridDim.x, id = blockIdx.x;
  const int L = (G % 8 == 0) ? (id % 8) * (G / 8) + id / 8 : id;
  const int ktile = L % a.ktiles, slice = L / a.ktiles;
  const int kbase = ktile * NW * CW + wave * CW;
  const int64_t rbeg = (int64_t)slice * a.rows_per_slice;
  const int64_t rend = (rbeg + a.rows_per_slice < N) ? rbeg + a.rows_per_slice : N;

  // ---- resident component operands: lane (li, g) holds component kbase+16ct+li, k-group g ----
  // 16-wave workgroups keep the augmented constants in LDS (row stride 40
  // bf16: conflict-free b128 reads, read once per block) to stay within 128
  // VGPRs; otherwise they are resident in VGPRs like the x·W' operands.
  constexpr bool AUG_LDS = NW >= 16;
  constexpr int AS = kAug + 8;
  __shared__ __align__(16) __bf16 augc[AUG_LDS ? NW * CW * AS : 8];
  bf16x8 whi[CT][ECH], wlo[CT][ECH], waug[AUG_LDS ? 1 : CT];
#pragma unroll
  for (int ct = 0; ct < CT; ++ct) {
    const int kk = kbase + 16 * ct + li;
    if (kk < K) {
      const size_t bk = (size_t)b * K + kk;
#pragma unroll
      for (int ec = 0; ec < ECH; ++ec) {
        whi[ct][ec] = ld16<bf16x8>(reinterpret_cast<const __bf16*>(a.w_hi) + bk * DP + 32 * ec + 8 * g);
        wlo[ct][ec] = ld16<bf16x8>(reinterpret_cast<const __bf16*>(a.w_lo) + bk * DP + 32 * ec + 8 * g);
      }
      const bf16x8 v = ld16<bf16x8>(reinterpret_cast<const __bf16*>(a.w_aug) + bk * kAug + 8 * g);
      if constexpr (AUG_LDS) *reinterpret_cast<bf16x8*>(&augc[(wave * CW + 16 * ct + li) * AS + 8 * g]) = v;
      else waug[ct] = v;
    } else {
#pragma unroll
      for (int s = 0; s < 8; ++s) {
#pragma unroll
        for (int ec = 0; ec < ECH; ++ec) { whi[ct][ec][s] = (__bf16)0.f; wlo[ct][ec][s] = (__bf16)0.f; }
        // padding component: C = -1e30 (column 6)
        const __bf16 v = (__bf16)((8 * g + s) == 6 ? -kHuge : 0.f);
        if constexpr (AUG_LDS) augc[(wave * CW + 16 * ct + li) * AS + 8 * g + s] = v;
        else waug[ct][s] = v;
      }
    }
  }

  f32x4 acc[STATS ? CT : 1][STATS ? JT : 1];
  if constexpr (STATS) {
#pragma unroll
    for (int ct = 0; ct < CT; ++ct)
#pragma unroll
      for (int jt = 0; jt < JT; ++jt) acc[ct][jt] = f32x4{0.f, 0.f, 0.f, 0.f};
  }

  // Constant augmented columns 8..31 of every staged row: [1 0 0 ...].
  for (int i = tid; i < NB * kBN * 3; i += NTHR) {
    const int row = i / 3, ch = 1 + i % 3;
    const uint4 w = make_uint4(ch == 1 ? pack2((__bf16)1.f, (__bf16)0.f) : 0u, 0u, 0u, 0u);
    *reinterpret_cast<uint4*>(xs + row * XS + DP + 8 * ch) = w;
  }
  __syncthreads();

  const __bf16* xb = reinterpret_cast<const __bf16*>(a.x) + (size_t)b * N * D;

  // ---- row-block loader: 16-byte chunks, PF per thread ----
  uint4 pf[PF];
  // Rows past the slice end read the last valid row (in bounds, no branch) and are zeroed.
  auto load_chunk = [&](int c, int64_t n0) -> uint4 {
    const int r = c / CPR, cc = (c % CPR) * 8;
    const int64_t n = n0 + r;
    const bool valid = n < rend;
    if (a.vec_ok) {
      const uint4 v = *reinterpret_cast<const uint4*>(xb + (size_t)(valid ? n : rend - 1) * D + cc);
      return valid ? v : make_uint4(0, 0, 0, 0);
    }
    if (!valid) return make_uint4(0, 0, 0, 0);
    union { uint4 u; __bf16 e[8]; } t;
#pragma unroll
    for (int j = 0; j < 8; ++j) t.e[j] = (cc + j < D) ? xb[(size_t)n * D + cc + j] : (__bf16)0.f;
    return t.u;
  };
  // Per-row extras fetched with the x chunks by each row's first chunk-lane:
  // the statistics / proba passes take the augmented chunk written by the
  // log-normaliser pass (rowaux) and the row's lse2.
  uint4 pa[PF];
  float pl[PF];
  float pt[TOPK ? PF : 1];
  int pti[TOPK ? PF : 1];
  auto fetch = [&](int64_t n0) {
#pragma unroll
    for (int i = 0; i < PF; ++i) {
      const int c = tid + i * NTHR;
      if (NCH % NTHR == 0 || c < NCH) {
        pf[i] = load_chunk(c, n0);
        if constexpr (!LSE) {
          const int64_t n = n0 + c / CPR;
          const size_t o = (size_t)b * N + (n < rend ? n : rend - 1);
          if (c % CPR == 0) {
            if constexpr (AUX) pa[i] = a.rowaux[o];
            pl[i] = (n < rend) ? a.lse2[o] : kHuge;
            if constexpr (TOPK) {
              pt[i] = (n < rend) ? a.thr2[o] : kHuge;
              pti[i] = (n < rend) ? a.thr_idx[o] : -1;
            }
          }
        }
      }
    }
  };
  // Stages the prefetched block into buffer `buf`: x, and columns 0..7 of the
  // augmented chunk (columns 8..31 are constant and written once).
  auto stash = [&](int buf, int64_t n0) {
#pragma unroll
    for (int i = 0; i < PF; ++i) {
      const int c = tid + i * NTHR;
      if (NCH % NTHR == 0 || c < NCH) {
        const int r = c / CPR, cc = c % CPR;
        const uint4 raw = pf[i];
        __bf16* row = xs + buf * kBN * XS + r * XS;
        *reinterpret_cast<uint4*>(row + 8 * cc) = raw;
        if constexpr (LSE || !AUX) {
          union { uint4 u; __bf16 e[8]; } t;
          t.u = raw;
          float q = 0.f;
#pragma unroll
          for (int j = 0; j < 8; ++j) {
            const float v = (float)t.e[j];
            q = fmaf(v, v, q);
          }
          q = group_sum<CPR>(q);
          if (cc == 0) {
            __bf16 h, m, l;
            split3(q, h, m, l);
            const uint4 w = make_uint4(pack2(h, m), pack2(l, h), pack2(m, h), pack2((__bf16)1.f, (__bf16)1.f));
            *reinterpret_cast<uint4*>(row + DP) = w;
            if constexpr (LSE && AUX) {
              const int64_t n = n0 + r;
              if (n < rend) a.rowaux[(size_t)b * N + n] = w;
            }
          }
        } else {
          if (cc == 0) *reinterpret_cast<uint4*>(row + DP) = pa[i];
        }
        if constexpr (!LSE) {
          if (cc == 0) lse_s[buf * kBN + r] = pl[i];
        }
        if constexpr (TOPK) {
          if (cc == 0) {
            thr_s[buf * kBN + r] = pt[i];
            thri_s[buf * kBN + r] = pti[i];
          }
        }
      }
    }
  };

  // Cross-wave merge of one block's per-row (max, sum[, argmax]) partials.
  auto combine_out = [&](int pb, int64_t n0) {
    if constexpr (LSE) {
      if (tid < kBN * NW) {
        const int r = tid / NW, w = tid % NW;
        const int o = (pb * NW + w) * RS + r;
        const float mw = red_m[o], sw = red_s[o];
        const float M = group_max<NW>(mw);
        const float t = group_sum<NW>(sw * fast_exp2(mw - M));
        int idx = 0;
        if constexpr (WANT_IDX) idx = group_min_i<NW>((mw == M) ? red_i[o] : 0x7fffffff);
        const int64_t n = n0 + r;
        if (w == 0 && n < rend) {
          const size_t og = ((size_t)ktile * a.B + b) * N + n;
          reinterpret_cast<float2*>(a.part_ms)[og] = make_float2(M, t);
          if constexpr (WANT_IDX) a.part_idx[og] = idx;
        }
      }
    }
  };

  // E-GEMM of staged block bx over row tiles h (rows 16h .. 16h+15).  LSE:
  // C = W·φᵀ (lane: 4 components of row 16h + li).  Otherwise C = φ·Wᵀ (lane:
  // rows 16h + 4g + v of component li).  Both read consecutive rows per lane
  // group, which the row stride keeps free of bank conflicts.
  struct Acc { f32x4 t[CT][2]; };
  auto wa = [&](int ct) -> bf16x8 {
    if constexpr (AUG_LDS) return ld16<bf16x8>(&augc[(wave * CW + 16 * ct + li) * AS + 8 * g]);
    else return waug[ct];
  };
  struct Frag { bf16x8 x[ECH + 1][2]; };          // [chunk (last = augmented)][row tile]
  auto load_frags = [&](int bx) -> Frag {
    Frag F;
    const __bf16* xr = xs + bx * kBN * XS;
#pragma unroll
    for (int h = 0; h < 2; ++h) {
      const __bf16* p = xr + (16 * h + li) * XS + 8 * g;
#pragma unroll
      for (int ec = 0; ec <= ECH; ++ec) F.x[ec][h] = ld16<bf16x8>(p + 32 * ec);
    }
    return F;
  };
  auto egemm = [&](const Frag& F) -> Acc {
    Acc A;
    auto mm = [&](const bf16x8& w, const bf16x8& x, const f32x4& c) {
      return LSE ? mfma_bf16(w, x, c) : mfma_bf16(x, w, c);
    };
#pragma unroll
    for (int ct = 0; ct < CT; ++ct)
#pragma unroll
      for (int h = 0; h < 2; ++h) A.t[ct][h] = mm(wa(ct), F.x[ECH][h], f32x4{0.f, 0.f, 0.f, 0.f});
    // consecutive MFMAs write different accumulators (no back-to-back dependency)
#pragma unroll
    for (int ec = 0; ec < ECH; ++ec) {
#pragma unroll
      for (int ct = 0; ct < CT; ++ct)
#pragma unroll
        for (int h = 0; h < 2; ++h) A.t[ct][h] = mm(whi[ct][ec], F.x[ec][h], A.t[ct][h]);
#pragma unroll
      for (int ct = 0; ct < CT; ++ct)
#pragma unroll
        for (int h = 0; h < 2; ++h) A.t[ct][h] = mm(wlo[ct][ec], F.x[ec][h], A.t[ct][h]);
    }
    return A;
  };

  // E-GEMM loading one k-chunk of operands at a time (fewer live registers).
  auto egemm_direct = [&](int bx) -> Acc {
    Acc A;
    const __bf16* xr = xs + bx * kBN * XS + li * XS + 8 * g;
    auto mm = [&](const bf16x8& w, const bf16x8& x, const f32x4& c) {
      return LSE ? mfma_bf16(w, x, c) : mfma_bf16(x, w, c);
    };
#pragma unroll
    for (int h = 0; h < 2; ++h) {
      const bf16x8 xa = ld16<bf16x8>(xr + 16 * h * XS + DP);
#pragma unroll
      for (int ct = 0; ct < CT; ++ct) A.t[ct][h] = mm(wa(ct), xa, f32x4{0.f, 0.f, 0.f, 0.f});
    }
#pragma unroll
    for (int ec = 0; ec < ECH; ++ec) {
      bf16x8 xv[2];
#pragma unroll
      for (int h = 0; h < 2; ++h) xv[h] = ld16<bf16x8>(xr + 16 * h * XS + 32 * ec);
#pragma unroll
      for (int ct = 0; ct < CT; ++ct)
#pragma unroll
        for (int h = 0; h < 2; ++h) A.t[ct][h] = mm(whi[ct][ec], xv[h], A.t[ct][h]);
#pragma unroll
      for (int ct = 0; ct < CT; ++ct)
#pragma unroll
        for (int h = 0; h < 2; ++h) A.t[ct][h] = mm(wlo[ct][ec], xv[h], A.t[ct][h]);
    }
    return A;
  };

  // lse2 of this lane's rows 16h + 4g + v (statistics / proba passes), read
  // before the next block's E-GEMM operands so the exponentials can start early.
  auto load_lse = [&](int bx, f32x4& ls0, f32x4& ls1) {
    if constexpr (!LSE) {
      ls0 = ld16<f32x4>(&lse_s[bx * kBN + 4 * g]);
      ls1 = ld16<f32x4>(&lse_s[bx * kBN + 16 + 4 * g]);
    }
  };
  auto epilogue = [&](const Acc& A, const f32x4& ls0, const f32x4& ls1, int bx, int pb, int64_t n0) {
    if constexpr (LSE) {
#pragma unroll
      for (int nt = 0; nt < 2; ++nt) {
        const int r = 16 * nt + li;
        float m = fmaxf(fmaxf(fmaxf(A.t[0][nt][0], A.t[0][nt][1]), fmaxf(A.t[0][nt][2], A.t[0][nt][3])),
                        fmaxf(fmaxf(A.t[1][nt][0], A.t[1][nt][1]), fmaxf(A.t[1][nt][2], A.t[1][nt][3])));
        int idx = 0x7fffffff;
        if constexpr (WANT_IDX) {
          // first component (lowest index) of this lane that attains the lane max
#pragma unroll
          for (int ct = CT - 1; ct >= 0; --ct)
#pragma unroll
            for (int v = 3; v >= 0; --v)
              if (A.t[ct][nt][v] == m) idx = kbase + 16 * ct + 4 * g + v;
        }
        const float lm = m;
        m = lanes_op<32, true>(lanes_op<16, true>(m));
        if constexpr (WANT_IDX) {
          idx = (lm == m) ? idx : 0x7fffffff;
          idx = lanes_min_i<32>(lanes_min_i<16>(idx));
        }
        float s = 0.f;
#pragma unroll
        for (int ct = 0; ct < CT; ++ct)
#pragma unroll
          for (int v = 0; v < 4; ++v) s += fast_exp2(A.t[ct][nt][v] - m);
        s = lanes_op<32, false>(lanes_op<16, false>(s));
        if (g == 0) {
          const int o = (pb * NW + wave) * RS + r;
          red_m[o] = m;
          red_s[o] = s;
          if constexpr (WANT_IDX) red_i[o] = idx;
        }
      }
    } else if constexpr (STATS) {
      bf16x8 ar[CT];
      if constexpr (TOPK) {
        // Only each row's top k (logit descending, then lower index) get mass;
        // lane (li, g) holds component kbase + 16ct + li of rows 4g + v and 16 + 4g + v.
        const f32x4 t0 = ld16<f32x4>(&thr_s[bx * kBN + 4 * g]);
        const f32x4 t1 = ld16<f32x4>(&thr_s[bx * kBN + 16 + 4 * g]);
        typedef int i32x4 __attribute__((ext_vector_type(4)));
        const i32x4 i0 = ld16<i32x4>(&thri_s[bx * kBN + 4 * g]);
        const i32x4 i1 = ld16<i32x4>(&thri_s[bx * kBN + 16 + 4 * g]);
#pragma unroll
        for (int ct = 0; ct < CT; ++ct) {
          const int kk = kbase + 16 * ct + li;
#pragma unroll
          for (int v = 0; v < 4; ++v) {
            const float l0 = A.t[ct][0][v], l1 = A.t[ct][1][v];
            // (hard: the one component thr_idx, by index, with r = 1 exactly)
            const bool k0 = a.hard ? kk == i0[v] : (l0 > t0[v] || (l0 == t0[v] && kk <= i0[v]));
            const bool k1 = a.hard ? kk == i1[v] : (l1 > t1[v] || (l1 == t1[v] && kk <= i1[v]));
            ar[ct][v] = (__bf16)(k0 ? (a.hard ? 1.f : fast_exp2(l0 - ls0[v])) : 0.f);
            ar[ct][4 + v] = (__bf16)(k1 ? (a.hard ? 1.f : fast_exp2(l1 - ls1[v])) : 0.f);
          }
        }
      } else {
#pragma unroll
        for (int ct = 0; ct < CT; ++ct)
#pragma unroll
          for (int v = 0; v < 4; ++v) {
            ar[ct][v] = (__bf16)fast_exp2(A.t[ct][0][v] - ls0[v]);
            ar[ct][4 + v] = (__bf16)fast_exp2(A.t[ct][1][v] - ls1[v]);
          }
      }
      // M-GEMM B operand ψ[k][feature 16jt + li] for k = 8g + 4h + j (data row
      // 16h + 4g + j) straight from the staged rows with the transposing LDS
      // read: in each 16-lane group, lane L supplies the 8-byte chunk of row
      // 4g + L/4 (+16), columns 16jt + 4(L%4) .. +3, and receives column li of
      // the four rows.
      const __bf16* xr = xs + bx * kBN * XS + (4 * g + (li >> 2)) * XS + 4 * (li & 3);
#pragma unroll
      for (int jt = 0; jt < JT; ++jt) {
        typedef short v4s __attribute__((ext_vector_type(4)));
        const v4s lo = __builtin_amdgcn_ds_read_tr16_b64_v4i16(
            (__attribute__((address_space(3))) v4s*)(xr + 16 * jt));
        const v4s hi = __builtin_amdgcn_ds_read_tr16_b64_v4i16(
            (__attribute__((address_space(3))) v4s*)(xr + 16 * XS + 16 * jt));
        const bf16x8 bq = __builtin_bit_cast(bf16x8, __builtin_shufflevector(lo, hi, 0, 1, 2, 3, 4, 5, 6, 7));
#pragma unroll
        for (int ct = 0; ct < CT; ++ct) acc[ct][jt] = mfma_bf16(ar[ct], bq, acc[ct][jt]);
      }
    } else {  // MODE_PROBA
#pragma unroll
      for (int ct = 0; ct < CT; ++ct) {
        const int kk = kbase + 16 * ct + li;
        if (kk < K) {
#pragma unroll
          for (int h = 0; h < 2; ++h)
#pragma unroll
            for (int v = 0; v < 4; ++v) {
              const int64_t n = n0 + 16 * h + 4 * g + v;
              if (n < rend)
                a.proba[((size_t)b * N + n) * K + kk] =
                    a.raw_logits ? A.t[ct][h][v] : fast_exp2(A.t[ct][h][v] - (h ? ls1[v] : ls0[v]));
            }
        }
      }
    }
  };

  // Issue order for one iteration's E-GEMM (next block) and epilogue (this
  // block), which form one basic block: each MFMA is followed by VALU work of
  // the epilogue so that the exponentials execute while the matrix core is busy
  // (a wave issues in order; back-to-back MFMAs would leave the VALU idle).
  constexpr int kEMfma = CT * 2 * (2 * ECH + 1);
  auto interleave = [&]() {
    constexpr int kMask_VALU = 0x002, kMask_MFMA = 0x008, kMask_DSR = 0x100;
#pragma unroll
    for (int i = 0; i < kEMfma; ++i) {
      __builtin_amdgcn_sched_group_barrier(kMask_MFMA, 1, 0);
      __builtin_amdgcn_sched_group_barrier(kMask_VALU, LSE ? 2 : 1, 0);
      if (STATS && i < 2 * JT) __builtin_amdgcn_sched_group_barrier(kMask_DSR, 1, 0);  // ψ operands
    }
    if constexpr (STATS) {
#pragma unroll
      for (int j = 0; j < CT * JT; ++j) {
        __builtin_amdgcn_sched_group_barrier(kMask_MFMA, 1, 0);
        __builtin_amdgcn_sched_group_barrier(kMask_VALU, 1, 0);
      }
    }
  };

  // ---- main loop: one barrier per block; loader two blocks ahead over three buffers ----
  const int nblk = (rend > rbeg) ? (int)((rend - rbeg + kBN - 1) / kBN) : 0;
  if (nblk > 0) { fetch(rbeg); stash(0, rbeg); }
  if (nblk > 1) { fetch(rbeg + kBN); stash(1, rbeg + kBN); }
  __syncthreads();
  // With 16 waves there are no registers for a second accumulator set: the
  // E-GEMM and epilogue of a block run back to back, and the other waves of
  // the SIMD fill the gaps.
  constexpr bool PIPE = NW < 16 && !TOPK;   // (the approximate pass skips the pipeline: fewer registers)
  Acc cur;
  if (PIPE && nblk > 0) cur = egemm(load_frags(0));
  int bx = 0;
  for (int ib = 0; ib < nblk; ++ib) {
    const int pb = ib & 1;
    const int b1 = (bx == NB - 1) ? 0 : bx + 1;   // buffer of block ib+1
    const int b2 = (b1 == NB - 1) ? 0 : b1 + 1;   // buffer of block ib+2
    const int64_t n0 = rbeg + (int64_t)ib * kBN;
    const bool ahead = ib + 2 < nblk;
    if (ahead) fetch(n0 + 2 * kBN);
    if (ib > 0) combine_out(pb ^ 1, n0 - kBN);
    // Block ib+1's MFMAs run under block ib's epilogue (the last iteration reads a
    // stale in-bounds buffer and discards the result).
    f32x4 ls0, ls1;
    load_lse(bx, ls0, ls1);
    if constexpr (PIPE) {
      const Acc nxt = egemm(load_frags(b1));
      epilogue(cur, ls0, ls1, bx, pb, n0);
      interleave();
      cur = nxt;
    } else {
      epilogue(egemm_direct(bx), ls0, ls1, bx, pb, n0);
    }
    if (ahead) stash(b2, n0 + 2 * kBN);
    __syncthreads();
    bx = b1;
  }
  if (nblk > 0) combine_out((nblk - 1) & 1, rbeg + (int64_t)(nblk - 1) * kBN);

  if constexpr (STATS) {
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

template <int DP, int NW>
static int launch_sph_bf16_nw(int mode, const TileArgs& a, dim3 grid, hipStream_t s) {
  const dim3 block(64 * NW);
  switch (mode) {
    case MODE_LSE: sph_bf16_kernel<DP, NW, MODE_LSE><<<grid, block, 0, s>>>(a); break;
    case MODE_LSE_IDX: sph_bf16_kernel<DP, NW, MODE_LSE_IDX><<<grid, block, 0, s>>>(a); break;
    case MODE_STATS: sph_bf16_kernel<DP, NW, MODE_STATS><<<grid, block, 0, s>>>(a); break;
    case MODE_PROBA: sph_bf16_kernel<DP, NW, MODE_PROBA><<<grid, block, 0, s>>>(a); break;
    case MODE_STATS_TOPK: sph_bf16_kernel<DP, NW, MODE_STATS_TOPK><<<grid, block, 0, s>>>(a); break;
    default: return -1;
  }
  return 0;
}

template <int DP>
static int launch_sph_bf16_dp(int nw, int mode, const TileArgs& a, dim3 grid, hipStream_t s) {
  switch (nw) {
    case 2: if constexpr (DP < 128) return launch_sph_bf16_nw<DP, 2>(mode, a, grid, s); else return -1;
    case 4: if constexpr (DP < 128) return launch_sph_bf16_nw<DP, 4>(mode, a, grid, s); else return -1;
    case 8: return launch_sph_bf16_nw<DP, 8>(mode, a, grid, s);
    case 16:  // plain log-normaliser pass at D = 128 only
      if constexpr (DP == 128) {
        if (mode == MODE_LSE) { sph_bf16_kernel<DP, 16, MODE_LSE><<<grid, dim3(1024), 0, s>>>(a); return 0; }
      }
      return -1;
    default: return -1;
  }
}

int launch_sph_bf16(int dp, int nw, int mode, const TileArgs& a, dim3 grid, hipStream_t s) {
  switch (dp) {
    case 32: return launch_sph_bf16_dp<32>(nw, mode, a, grid, s);
    case 64: return launch_sph_bf16_dp<64>(nw, mode, a, grid, s);
    case 128: return launch_sph_bf16_dp<128>(nw, mode, a, grid, s);
    default: return -1;
  }
}

}  // namespace gx
