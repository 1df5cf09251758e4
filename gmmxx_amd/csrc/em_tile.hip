// The GMM EM tile kernel for gfx950 (CDNA4).
//
// One workgroup owns a tile of KT = nwaves * CW mixture components and a
// contiguous slice of rows of one batch.  Each wave keeps the E-step operand W
// for its CW components resident in VGPRs as MFMA fragments for the whole
// launch.  Rows are processed in blocks of 32 with one barrier per block: a
// later block's x is fetched into registers before the current block is
// computed and stashed into a free LDS buffer after it; the loading threads
// build ‖x‖² and the xxᵀ products from their own registers.  For bf16 the
// transposed M-step operand ψᵀ is built from the staged rows one block ahead
// (the loader then runs two blocks ahead over three row buffers), which keeps
// the LDS traffic free of bank conflicts.
//
//   MODE_LSE / MODE_LSE_IDX
//               E-GEMM in "component rows" orientation (C = W·φᵀ), so a lane
//               holds 4·CW/16 components of one data row; per-row max, scaled
//               sum (and, for _IDX, first-index argmax) are reduced across
//               lanes with two shuffles and across waves through LDS, and
//               written as one partial per row and component tile.
//   MODE_STATS  E-GEMM in "data rows" orientation (C = φ·Wᵀ); the epilogue turns
//               logits into responsibilities r = 2^(l2 - lse2) in registers and
//               feeds them directly as the A operand of the M-GEMM acc += rᵀ·ψ,
//               so the (B, N, K) responsibility matrix never exists.  Each
//               workgroup writes one partial statistics tile.
//   MODE_PROBA  Same epilogue; r is written out (predict_proba needs it), or
//               with raw_logits the log2 logits themselves (approximate EM).
//   MODE_STATS_TOPK
//               MODE_STATS restricted to each row's top k components: a
//               logit keeps its responsibility iff it ranks above the row's
//               threshold (value, then lower index), else contributes 0.  The
//               E-GEMM and logit arithmetic are those of MODE_PROBA, so the
//               recomputed logits equal the ones the threshold was chosen from.
//   MODE_STATS_LSE
//               MODE_STATS when the workgroup holds all K components (one
//               component tile): each wave reduces its rows' (max, sum) over
//               its components with DPP, the waves' partials meet in LDS after
//               one barrier, and every wave merges them for its own use, so the
//               EM iteration needs no separate log-normaliser pass.  The
//               workgroup also writes its rows' log-likelihood sum.
//   MODE_PROBA_LSE
//               MODE_PROBA with the same in-workgroup log-normalisers.
//
// Logits are kept in log2 units (l2 = l·log2 e) so exp2 maps to v_exp_f32:
//   l2 = A_k·S + (a_k·rowq_n + C_k)
// with S the E-GEMM output, rowq_n the per-row term (‖x‖² spherical, xᵀPx
// tied, 0 otherwise) and (A_k, a_k, C_k) per-component constants.  The
// reference clamps the squared distance at 0 before scaling; that clamp only
// removes negative rounding residue and is dropped here.
// bf16 inputs multiply exact bf16 x against a hi/lo bf16 split of the fp32
// operand, which keeps the cross term at fp32-oracle noise level.

#include <atomic>
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

typedef float f32x2 __attribute__((ext_vector_type(2)));
typedef __bf16 bf16x2 __attribute__((ext_vector_type(2)));

// (a, b) split into three bf16 parts each, v = v1 + v2 + v3 exactly; part p of
// both values packed into qp (a in the low half).
__device__ __forceinline__ void split3x2(float a, float b, uint32_t& q1, uint32_t& q2, uint32_t& q3) {
  const f32x2 v = f32x2{a, b};
  const bf16x2 h = __builtin_convertvector(v, bf16x2);
  const f32x2 r = v - __builtin_convertvector(h, f32x2);
  const bf16x2 m = __builtin_convertvector(r, bf16x2);
  const bf16x2 l = __builtin_convertvector(r - __builtin_convertvector(m, f32x2), bf16x2);
  q1 = __builtin_bit_cast(uint32_t, h);
  q2 = __builtin_bit_cast(uint32_t, m);
  q3 = __builtin_bit_cast(uint32_t, l);
}

typedef short v4s __attribute__((ext_vector_type(4)));

// Transposing LDS read: in each 16-lane group, lane L supplies the address of
// an 8-byte chunk; lane i receives word (i % 4) of the chunks of lanes 4j + i/4.
__device__ __forceinline__ v4s tr16(const __bf16* p) {
  return __builtin_amdgcn_ds_read_tr16_b64_v4i16((__attribute__((address_space(3))) v4s*)p);
}
__device__ __forceinline__ bf16x8 cat_v4s(v4s lo, v4s hi) {
  return __builtin_bit_cast(bf16x8, __builtin_shufflevector(lo, hi, 0, 1, 2, 3, 4, 5, 6, 7));
}

// Lane maxima start at this floor instead of -inf so merges need no guards;
// invalid components still contribute exp2(-inf - m) = 0.
constexpr float kLogFloor = -1e30f;

template <int CTRL>
__device__ __forceinline__ float dpp(float v) {
  return __int_as_float(__builtin_amdgcn_update_dpp(0, __float_as_int(v), CTRL, 0xF, 0xF, false));
}

// Sum over groups of G consecutive lanes (G = 1, 2, 4, 8, 16, 32), result in every lane.
template <int G>
__device__ __forceinline__ float group_sum(float v) {
  if constexpr (G >= 2) v += dpp<0xB1>(v);    // quad_perm [1,0,3,2]: lane ^ 1
  if constexpr (G >= 4) v += dpp<0x4E>(v);    // quad_perm [2,3,0,1]: lane ^ 2
  if constexpr (G >= 8) v += dpp<0x141>(v);   // row_half_mirror: the other quad of 8
  if constexpr (G >= 16) v += dpp<0x140>(v);  // row_mirror: the other half of 16
  if constexpr (G >= 32) {
    const auto t = __builtin_amdgcn_permlane16_swap(__float_as_uint(v), __float_as_uint(v), false, false);
    v = __uint_as_float(t[0]) + __uint_as_float(t[1]);
  }
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
  auto d = [](int x, auto ctrl) { return __builtin_amdgcn_update_dpp(0, x, decltype(ctrl)::value, 0xF, 0xF, false); };
  if constexpr (G >= 2) v = min(v, d(v, std::integral_constant<int, 0xB1>{}));
  if constexpr (G >= 4) v = min(v, d(v, std::integral_constant<int, 0x4E>{}));
  if constexpr (G >= 8) v = min(v, d(v, std::integral_constant<int, 0x141>{}));
  return v;
}

// Value combined with its partner lane l ^ 16 (OFF = 16) or l ^ 32 (OFF = 32) by OP, no LDS.
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

// Packed upper-triangle index -> (d, e) for the full covariance (DP = 16).

// (max, Σ s·2^(m - max)) over the nw (1, 2 or 4) wave partials of a row,
// unrolled for each count.
template <int NW>
__device__ __forceinline__ void merge_waves_n(const float* rm, const float* rsum, float& M, float& S) {
  float m[NW];
#pragma unroll
  for (int w = 0; w < NW; ++w) m[w] = rm[w];
  M = m[0];
#pragma unroll
  for (int w = 1; w < NW; ++w) M = fmaxf(M, m[w]);
  S = 0.f;
#pragma unroll
  for (int w = 0; w < NW; ++w) S += rsum[w] * fast_exp2(m[w] - M);
}
__device__ __forceinline__ void merge_waves(int nw, const float* rm, const float* rsum, float& M, float& S) {
  switch (nw) {
    case 4: merge_waves_n<4>(rm, rsum, M, S); break;
    case 2: merge_waves_n<2>(rm, rsum, M, S); break;
    default: merge_waves_n<1>(rm, rsum, M, S); break;
  }
}

template <int COV, typename XT, int DP, int CW, int MODE>
__global__ __launch_bounds__(512) void em_tile_kernel(TileArgs a) {
  constexpr bool BF = sizeof(XT) == 2;
  constexpr bool LSE = (MODE == MODE_LSE || MODE == MODE_LSE_IDX);
  constexpr bool WANT_IDX = MODE == MODE_LSE_IDX;
  constexpr bool SLSE = MODE == MODE_STATS_LSE || MODE == MODE_PROBA_LSE;
  constexpr bool XCH = MODE == MODE_STATS_XCH;
  constexpr bool STATS = MODE == MODE_STATS || MODE == MODE_STATS_TOPK || MODE == MODE_STATS_LSE || XCH;
  constexpr bool TOPK = MODE == MODE_STATS_TOPK;
  using Dm = Dims<COV, DP, BF>;
  constexpr int EP = Dm::EP, JP = Dm::JP, J = Dm::J, S = Dm::S;
  constexpr int CT = CW / 16;
  constexpr int ECH = BF ? EP / 32 : EP / 16;
  constexpr int JT = JP / 16;
  constexpr int VEC = 16 / sizeof(XT);                   // elements per 16-byte chunk
  constexpr int CPR = DP / VEC;                          // chunks per row
  constexpr int NCH = kBN * CPR;                         // chunks per row block
  constexpr int PF = (NCH + 511) / 512;                  // prefetched chunks per thread at 512 threads
  constexpr bool PSI_LDS = BF && (MODE == MODE_STATS || MODE == MODE_STATS_TOPK);  // materialised ψᵀ (bf16 spherical)
  // Block i+1's E-GEMM issued ahead of block i's epilogue: kept for the bf16
  // path only.  The fp32 (split-bf16) passes measured equal or faster without
  // it (C3 3.45 vs 3.47 ms, C4 0.87 vs 0.93 ms): MFMA and VALU time add up on
  // this machine, and the second accumulator set only costs registers.
  constexpr bool PIPE = BF && COV != FULL;
  constexpr int PD = PIPE ? 2 : 1;                       // loader runs PD blocks ahead
  // Staged-row buffers: the loader fills one while the waves read the other, one
  // barrier per block.  Full covariance stages three 176-column parts per row and
  // keeps a single buffer (a second barrier per block) so that two workgroups of
  // two waves fit a CU's LDS twice over.
  // The exchange pass keeps block i-1 staged for its M-GEMM while block i is
  // computed and block i+1 loads: one more buffer.
  constexpr int NB = (COV == FULL) ? 1 : PD + 1 + (XCH ? 1 : 0);
  constexpr int XS = DP + (BF ? 8 : 4);                  // staged-row stride, elements
  constexpr int QS = kBN + 8;                            // ψᵀ row stride, bf16 elements
  using FT = typename std::conditional<BF, __bf16, float>::type;
  using WF = typename std::conditional<BF, bf16x8, f32x4>::type;
  static_assert(NCH % 64 == 0, "row block must split into whole waves of chunks");
  // Split-bf16 E-GEMM (fp32 x, log-normaliser passes): the E-step features φ and W
  // are each split into three bf16 parts (v = v1 + v2 + v3 exactly) and the
  // product runs as six 16x16x32 bf16 MFMAs per 32-deep k-step, keeping every
  // cross term down to 2^-24 relative -- fp32 accuracy at 6/16 of the cost of
  // the fp32 MFMA.  φ parts are staged once per block for all waves.
  // Every pass of a shape uses the same E-GEMM, so all of them see identical logits
  // (off for diag at D = 128: its three staged φ parts would not fit the LDS).
  constexpr bool X3 = !BF && !(COV == DIAG && DP >= 128);
  constexpr int X3K = EP / 32;                           // k-steps of the split E-GEMM
  constexpr int EPS = EP + 16;                           // split-φ row stride (s ≡ 8 or 24 mod 32 dwords)
  constexpr int X3P = NB * kBN * EPS;                    // one part, all buffers
  // Wide statistics passes keep W's third part in LDS (per wave, in the exact
  // per-lane fragment order) to stay within the register file.
  constexpr bool W3L = X3 && STATS && EP >= 128 && COV != FULL;

  __shared__ __align__(16) XT xs[(COV == FULL || X3) ? 8 : NB * kBN * XS];
  __shared__ __align__(16) __bf16 phx[X3 ? 3 * X3P : 8];
  __shared__ __align__(16) bf16x8 w3s[W3L ? 8 * (CW / 16) * X3K * 64 : 1];   // [wave][ct][ec][lane]
  __shared__ __align__(16) FT psiT[PSI_LDS ? 2 * JP * QS : 8];
  __shared__ float rowq_s[NB * kBN];
  __shared__ float lse_s[NB * kBN];
  __shared__ float thr_s[TOPK ? NB * kBN : 1];     // top-k threshold logit and index per row
  __shared__ int thri_s[TOPK ? NB * kBN : 1];
  __shared__ float red_m[(LSE || SLSE || XCH) ? 2 * kBN * 8 : 1];   // [parity][row][wave]
  __shared__ float red_s[(LSE || SLSE || XCH) ? 2 * kBN * 8 : 1];
  __shared__ __align__(16) float lsw[(SLSE || XCH) ? 8 * kBN : 4];   // [wave][row] merged log-normalisers
  __shared__ int red_i[WANT_IDX ? 2 * kBN * 8 : 1];

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
  // (split-bf16: w3[p][ct][ec] = part p of W[16ct + li][32ec + 8g .. +7])
  bf16x8 w3[X3 ? (W3L ? 2 : 3) : 1][X3 ? CT : 1][X3 ? X3K : 1];
  if constexpr (X3) {
#pragma unroll
    for (int ct = 0; ct < CT; ++ct) {
      const int kk = kbase + 16 * ct + li;
#pragma unroll
      for (int ec = 0; ec < X3K; ++ec) {
        f32x4 lo4 = f32x4{0.f, 0.f, 0.f, 0.f}, hi4 = lo4;
        if (kk < K) {
          const float* wp = reinterpret_cast<const float*>(a.w_hi) + ((size_t)b * K + kk) * EP + 32 * ec + 8 * g;
          lo4 = ld16<f32x4>(wp);
          hi4 = ld16<f32x4>(wp + 4);
        }
#pragma unroll
        for (int j = 0; j < 8; ++j) {
          const float v = j < 4 ? lo4[j] : hi4[j - 4];
          const __bf16 p1 = (__bf16)v;
          const float r1 = v - (float)p1;
          const __bf16 p2 = (__bf16)r1;
          w3[0][ct][ec][j] = p1;
          w3[1][ct][ec][j] = p2;
          if constexpr (W3L) w3s[((wave * CT + ct) * X3K + ec) * 64 + lane][j] = (__bf16)(r1 - (float)p2);
          else w3[W3L ? 0 : 2][ct][ec][j] = (__bf16)(r1 - (float)p2);
        }
      }
    }
  }
  WF whi[X3 ? 1 : CT][X3 ? 1 : ECH];
  WF wlo[BF ? CT : 1][BF ? ECH : 1];
#pragma unroll
  for (int ct = 0; ct < (X3 ? 0 : CT); ++ct) {
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
  // Per-component (c, C): l2 = c*(rowq - 2S) + C (spherical, tied) or c*S + C (diag, full);
  // components past K get C = -inf.
  constexpr bool ROWQ = (COV == SPH || COV == TIED);
  const float2 kInvalid = make_float2(0.f, -INFINITY);
  float2 cS[CT];           // data-row orientation: component kbase + 16ct + li
  float2 cL[CT][4];        // component-row orientation: kbase + 16ct + 4g + v
#pragma unroll
  for (int ct = 0; ct < CT; ++ct) {
    const int k1 = kbase + 16 * ct + li;
    if (k1 < K) { const float4 c = a.cconst[(size_t)b * K + k1]; cS[ct] = make_float2(c.x, c.y); }
    else cS[ct] = kInvalid;
#pragma unroll
    for (int v = 0; v < 4; ++v) {
      const int k2 = kbase + 16 * ct + 4 * g + v;
      if (k2 < K) { const float4 c = a.cconst[(size_t)b * K + k2]; cL[ct][v] = make_float2(c.x, c.y); }
      else cL[ct][v] = kInvalid;
    }
  }
  auto logit = [&](float2 c, float S, float rq) -> float {
    if constexpr (ROWQ) return fmaf(c.x, fmaf(-2.f, S, rq), c.y);
    else return fmaf(c.x, S, c.y);
  };

  f32x4 acc[STATS ? CT : 1][STATS ? JT : 1];
  double ll_acc = 0.0;     // MODE_STATS_LSE, wave 0: Σ log2-normalisers of this workgroup's rows
  if constexpr (STATS) {
#pragma unroll
    for (int ct = 0; ct < CT; ++ct)
#pragma unroll
      for (int jt = 0; jt < JT; ++jt) acc[ct][jt] = f32x4{0.f, 0.f, 0.f, 0.f};
  }
  // Constant feature rows, written once for both buffers.
  if constexpr (PSI_LDS) {
    for (int i = tid; i < 2 * (JP - DP) * QS; i += nthr) {
      const int bufi = i / ((JP - DP) * QS), rem = i % ((JP - DP) * QS);
      const int j = DP + rem / QS;
      psiT[bufi * JP * QS + j * QS + rem % QS] = (FT)(j == DP ? 1.f : 0.f);
    }
  }
  if constexpr (X3) {
    constexpr int E = Dm::E;
    for (int i = tid; i < 3 * NB * kBN * (EP - E); i += nthr) {
      const int row = i / (EP - E), c = E + i % (EP - E);
      phx[row * EPS + c] = (__bf16)0.f;   // row runs over every part and buffer
    }
    // Augmented ψ columns EP..EP+15 (statistics pass): part 1 = [1 0 ...], parts 2, 3 = 0
    // (spherical rows put their ‖x‖² parts at EP+1 when staged).
    for (int i = tid; i < 3 * NB * kBN * 16; i += nthr) {
      const int row = i / 16, c = i % 16;
      phx[row * EPS + EP + c] = (__bf16)((c == 0 && row < NB * kBN) ? 1.f : 0.f);
    }
  }

  const XT* xb = reinterpret_cast<const XT*>(a.x) + (size_t)b * N * D;

  // ---- row-block loader ----
  uint4 pf[PF];
  auto load_chunk = [&](int c, int64_t n0) -> uint4 {
    const int r = c / CPR, cc = (c % CPR) * VEC;
    const int64_t n = n0 + r;
    if (n >= rend) return make_uint4(0, 0, 0, 0);
    if (a.vec_ok) return *reinterpret_cast<const uint4*>(xb + (size_t)n * D + cc);
    union { uint4 u; XT e[VEC]; } t;
#pragma unroll
    for (int j = 0; j < VEC; ++j) t.e[j] = (cc + j < D) ? xb[(size_t)n * D + cc + j] : (XT)0.f;
    return t.u;
  };
  auto fetch = [&](int64_t n0) {
#pragma unroll
    for (int i = 0; i < PF; ++i) {
      const int c = tid + i * nthr;
      if (c < NCH) pf[i] = load_chunk(c, n0);
    }
  };
  // Writes the block's staged rows and features into buffer `buf`.
  auto stash = [&](int buf, int64_t n0) {
    int i = 0;
    for (int c = tid; c < NCH; c += nthr, ++i) {          // uniform per wave (NCH % 64 == 0)
      const uint4 raw = (i < PF) ? pf[i < PF ? i : 0] : load_chunk(c, n0);
      const int r = c / CPR, cc = (c % CPR) * VEC;
      const int64_t n = n0 + r;
      union { uint4 u; XT e[VEC]; } t;
      t.u = raw;
      float v[VEC];
#pragma unroll
      for (int j = 0; j < VEC; ++j) v[j] = to_f32(t.e[j]);
      if constexpr (X3) {
        // φ features of these VEC columns, split into three bf16 parts.
        auto put3 = [&](int col, const float (&f)[VEC]) {
          uint32_t q1[VEC / 2], q2[VEC / 2], q3[VEC / 2];
#pragma unroll
          for (int j = 0; j < VEC; j += 2) split3x2(f[j], f[j + 1], q1[j / 2], q2[j / 2], q3[j / 2]);
          __bf16* base = phx + (buf * kBN + r) * EPS + col;
          *reinterpret_cast<uint2*>(base) = make_uint2(q1[0], q1[1]);
          *reinterpret_cast<uint2*>(base + X3P) = make_uint2(q2[0], q2[1]);
          *reinterpret_cast<uint2*>(base + 2 * X3P) = make_uint2(q3[0], q3[1]);
        };
        // NN (even) consecutive features from column col: 16-byte stores when the
        // run is a multiple of 8 (col is then a multiple of 8), else 4-byte stores.
        auto put3n = [&](int col, const auto& f) {
          constexpr int NN = sizeof(f) / sizeof(float);
          uint32_t q[3][NN / 2];
#pragma unroll
          for (int j = 0; j < NN; j += 2) split3x2(f[j], f[j + 1], q[0][j / 2], q[1][j / 2], q[2][j / 2]);
          __bf16* base = phx + (buf * kBN + r) * EPS + col;
#pragma unroll
          for (int p = 0; p < 3; ++p) {
            if constexpr (NN % 8 == 0) {
#pragma unroll
              for (int u = 0; u < NN / 8; ++u)
                *reinterpret_cast<uint4*>(base + p * X3P + 8 * u) =
                    make_uint4(q[p][4 * u], q[p][4 * u + 1], q[p][4 * u + 2], q[p][4 * u + 3]);
            } else {
#pragma unroll
              for (int u = 0; u < NN / 2; ++u) *reinterpret_cast<uint32_t*>(base + p * X3P + 2 * u) = q[p][u];
            }
          }
        };
        if constexpr (COV == DIAG) {
          float sq[VEC];
#pragma unroll
          for (int j = 0; j < VEC; ++j) sq[j] = v[j] * v[j];
          put3(cc, sq);
          put3(DP + cc, v);
        } else if constexpr (COV == FULL) {
          // φ = [xxᵀ products in full_feature order | x]: the row's four chunks sit
          // in a quad of lanes; this lane (chunk c = cc / 4) writes its diagonal
          // block, its chunk times chunk c+1, half of the pair {c, c+2} (rows
          // 2h, 2h+1 of the owner's 4x4 block, h = c / 2, owner c % 2) and its x
          // values: 38 features per lane, so no lane of the wave idles while
          // others form the pair blocks.
          static_assert(DP == 16 && VEC == 4 && CPR == 4, "full covariance runs at DP = 16");
          const int c = cc / VEC, q0 = lane & ~3;
          float w1[VEC], w2[VEC];
#pragma unroll
          for (int j = 0; j < VEC; ++j) {
            w1[j] = __shfl(v[j], q0 + ((c + 1) & 3));
            w2[j] = __shfl(v[j], q0 + ((c + 2) & 3));
          }
          float dg[10];
#pragma unroll
          for (int i = 0, t = 0; i < VEC; ++i)
#pragma unroll
            for (int j = i; j < VEC; ++j, ++t) dg[t] = v[i] * v[j];
          put3n(10 * c, dg);
          float o[16];
#pragma unroll
          for (int i = 0; i < VEC; ++i)
#pragma unroll
            for (int j = 0; j < VEC; ++j) o[4 * i + j] = v[i] * w1[j];
          put3n(40 + 16 * c, o);
          {
            // owner chunk a = c % 2 (rows i of the block), partner a + 2 (columns j);
            // lanes c < 2 hold a in v, lanes c >= 2 hold it in w2
            const int h = c >> 1;
            float p8[8];
#pragma unroll
            for (int ii = 0; ii < 2; ++ii)
#pragma unroll
              for (int j = 0; j < VEC; ++j) {
                const float own = h ? w2[2 + ii] : v[ii];   // row 2h + ii of chunk a
                const float par = h ? v[j] : w2[j];
                p8[4 * ii + j] = own * par;
              }
            put3n(104 + 16 * (c & 1) + 8 * h, p8);
          }
          put3(S + cc, v);
        } else {
          put3(cc, v);
        }
      }
      if constexpr (COV != FULL && !X3) {
        *reinterpret_cast<uint4*>(&xs[buf * kBN * XS + r * XS + cc]) = raw;
      }
      if constexpr (COV == SPH) {
        float q = 0.f;
#pragma unroll
        for (int j = 0; j < VEC; ++j) q = fmaf(v[j], v[j], q);
        q = group_sum<CPR>(q);
        if (cc == 0) rowq_s[buf * kBN + r] = q;
        if constexpr (X3 && STATS) {
          if (cc == 0) {
            uint32_t q1, q2, q3;
            split3x2(q, 0.f, q1, q2, q3);
            __bf16* at = phx + (buf * kBN + r) * EPS + EP + 1;
            *at = __builtin_bit_cast(__bf16, (uint16_t)q1);
            at[X3P] = __builtin_bit_cast(__bf16, (uint16_t)q2);
            at[2 * X3P] = __builtin_bit_cast(__bf16, (uint16_t)q3);
          }
        }
      } else if constexpr (COV == TIED) {
        // (no rowq: the EM iteration's logits leave the row constant xᵀPx out)
        if (cc == 0) rowq_s[buf * kBN + r] = (n < rend && a.rowq) ? a.rowq[(size_t)b * N + n] : 0.f;
      } else {
        if (cc == 0) rowq_s[buf * kBN + r] = 0.f;
      }
      if constexpr (!LSE && !SLSE && !XCH) {
        if (cc == 0) lse_s[buf * kBN + r] = (n < rend) ? a.lse2[(size_t)b * N + n] : INFINITY;
      }
      if constexpr (TOPK) {
        if (cc == 0) {
          thr_s[buf * kBN + r] = (n < rend) ? a.thr2[(size_t)b * N + n] : INFINITY;
          thri_s[buf * kBN + r] = (n < rend) ? a.thr_idx[(size_t)b * N + n] : -1;
        }
      }
    }
  };

  // Transposed M-step operand ψᵀ (bf16) from staged rows: each thread reads 8
  // rows of one column (consecutive lanes -> consecutive columns, no bank
  // conflicts) and writes one 16-byte chunk of a ψᵀ row.
  auto build_psi = [&](int bx, int pb) {
    if constexpr (PSI_LDS) {
      const XT* xr = xs + bx * kBN * XS;
      FT* pt = psiT + pb * JP * QS;
      for (int t = tid; t < DP * (kBN / 8); t += nthr) {
        const int j = t % DP, q = t / DP;
        bf16x8 v;
#pragma unroll
        for (int s8 = 0; s8 < 8; ++s8) v[s8] = xr[(8 * q + s8) * XS + j];
        *reinterpret_cast<bf16x8*>(&pt[j * QS + 8 * q]) = v;
      }
      if (tid < kBN) {
        const float q = rowq_s[bx * kBN + tid];
        const __bf16 hi = (__bf16)q;
        pt[(DP + 1) * QS + tid] = hi;
        pt[(DP + 2) * QS + tid] = (__bf16)(q - (float)hi);
      }
    }
  };

  // φ fragment (4 consecutive E-step features of staged row r), fp32 path.
  auto phi4 = [&](int buf, int r, int e0) -> f32x4 {
    if constexpr (COV == DIAG) {
      const int c = e0 < DP ? e0 : e0 - DP;
      f32x4 v = ld16<f32x4>(&xs[buf * kBN * XS + r * XS + c]);
      if (e0 < DP) v = v * v;
      return v;
    } else {
      return ld16<f32x4>(&xs[buf * kBN * XS + r * XS + e0]);
    }
  };
  // ψ element (M-step feature j of staged row r), fp32 path.
  auto psi1 = [&](int buf, int r, int j) -> float {
    const float* xr = reinterpret_cast<const float*>(xs) + buf * kBN * XS + r * XS;
    if (j < DP) return xr[j];
    if constexpr (COV == SPH) return j == DP ? 1.f : (j == DP + 1 ? rowq_s[buf * kBN + r] : 0.f);
    if constexpr (COV == DIAG) {
      if (j < 2 * DP) { const float t = xr[j - DP]; return t * t; }
      return j == 2 * DP ? 1.f : 0.f;
    }
    return j == DP ? 1.f : 0.f;  // tied
  };

  // Cross-wave merge of one block's per-row partials, written to global memory:
  // lane (row, wave) of the first 32*nw threads holds one partial; the nw
  // partials of a row sit in consecutive lanes and are reduced with DPP.
  auto combine_out = [&](int pb, int64_t n0) {
    if (tid < kBN * nw) {
      const int r = tid / nw, w = tid % nw;
      const int o = (pb * kBN + r) * 8 + w;
      const float mw = red_m[o], sw = red_s[o];
      float M;
      switch (nw) {
        case 1: M = mw; break;
        case 2: M = group_max<2>(mw); break;
        case 4: M = group_max<4>(mw); break;
        default: M = group_max<8>(mw); break;
      }
      float t = sw * fast_exp2(mw - M);
      int idx = 0;
      if constexpr (WANT_IDX) idx = (mw == M) ? red_i[o] : 0x7fffffff;
      switch (nw) {
        case 1: break;
        case 2: t = group_sum<2>(t); if (WANT_IDX) idx = group_min_i<2>(idx); break;
        case 4: t = group_sum<4>(t); if (WANT_IDX) idx = group_min_i<4>(idx); break;
        default: t = group_sum<8>(t); if (WANT_IDX) idx = group_min_i<8>(idx); break;
      }
      const int64_t n = n0 + r;
      if (w == 0 && n < rend) {
        const size_t og = ((size_t)ktile * a.B + b) * N + n;
        reinterpret_cast<float2*>(a.part_ms)[og] = make_float2(M, t);
        if constexpr (WANT_IDX) a.part_idx[og] = idx;
      }
    }
  };

  // E-GEMM of one staged block.  LSE modes: component-row orientation,
  // T[ct][nt] = W(16 comps) · φᵀ(16 rows).  Otherwise data-row orientation,
  // T[ct][rt] = φ(16 rows) · Wᵀ(16 comps); for bf16 tile rt's A-row i is data row
  // 8(i/4) + 4rt + i%4, so C-row 4g+v of tile rt is data row 8g + 4rt + v.
  struct Acc { f32x4 t[CT][2]; };
  auto egemm = [&](int bx) -> Acc {
    Acc A;
#pragma unroll
    for (int ct = 0; ct < CT; ++ct) { A.t[ct][0] = f32x4{0.f, 0.f, 0.f, 0.f}; A.t[ct][1] = A.t[ct][0]; }
    if constexpr (X3) {
      // Six products per k-step, the smallest first: W1φ3, W3φ1, W2φ2, W1φ2, W2φ1, W1φ1.
      // Full covariance sums the five correction products in an accumulator of
      // their own: its logits are differences of terms ~10^2 times larger, and
      // adding each small product to the large running sum would round it at
      // that sum's magnitude (five roundings per k-step instead of one).
      constexpr bool SPLIT = COV == FULL;
      Acc Bs;
      if constexpr (SPLIT)
#pragma unroll
        for (int ct = 0; ct < CT; ++ct) { Bs.t[ct][0] = A.t[ct][0]; Bs.t[ct][1] = A.t[ct][0]; }
#pragma unroll
      for (int ec = 0; ec < X3K; ++ec) {
        bf16x8 xv[3][2];
#pragma unroll
        for (int p = 0; p < 3; ++p)
#pragma unroll
          for (int h = 0; h < 2; ++h)
            xv[p][h] = ld16<bf16x8>(&phx[p * X3P + (bx * kBN + 16 * h + li) * EPS + 32 * ec + 8 * g]);
#pragma unroll
        for (int ct = 0; ct < CT; ++ct)
#pragma unroll
          for (int h = 0; h < 2; ++h) {
            // LSE: C = W·φᵀ (lane: components 4g + v of row li); otherwise C = φ·Wᵀ
            // (lane: rows 4g + v of component li), the M-GEMM's A-operand layout.
            auto mm = [&](const bf16x8& w, const bf16x8& x, const f32x4& c) {
              return LSE ? mfma_bf16(w, x, c) : mfma_bf16(x, w, c);
            };
            const bf16x8 wp3 = W3L ? w3s[((wave * CT + ct) * X3K + ec) * 64 + lane] : w3[W3L ? 0 : 2][ct][ec];
            f32x4& sm = SPLIT ? Bs.t[ct][h] : A.t[ct][h];
            sm = mm(w3[0][ct][ec], xv[2][h], sm);
            sm = mm(wp3, xv[0][h], sm);
            sm = mm(w3[1][ct][ec], xv[1][h], sm);
            sm = mm(w3[0][ct][ec], xv[1][h], sm);
            sm = mm(w3[1][ct][ec], xv[0][h], sm);
            A.t[ct][h] = mm(w3[0][ct][ec], xv[0][h], A.t[ct][h]);
          }
      }
      if constexpr (SPLIT)
#pragma unroll
        for (int ct = 0; ct < CT; ++ct) { A.t[ct][0] += Bs.t[ct][0]; A.t[ct][1] += Bs.t[ct][1]; }
      return A;
    } else {
#pragma unroll
    for (int ec = 0; ec < ECH; ++ec) {
      if constexpr (BF) {
        bf16x8 xv[2];
#pragma unroll
        for (int h = 0; h < 2; ++h) {
          const int row = LSE ? 16 * h + li : 8 * (li / 4) + 4 * h + (li % 4);
          xv[h] = ld16<bf16x8>(&xs[bx * kBN * XS + row * XS + 32 * ec + 8 * g]);
        }
#pragma unroll
        for (int ct = 0; ct < CT; ++ct)
#pragma unroll
          for (int h = 0; h < 2; ++h) {
            if constexpr (LSE) {
              A.t[ct][h] = mfma_bf16(whi[ct][ec], xv[h], A.t[ct][h]);
              A.t[ct][h] = mfma_bf16(wlo[ct][ec], xv[h], A.t[ct][h]);
            } else {
              A.t[ct][h] = mfma_bf16(xv[h], whi[ct][ec], A.t[ct][h]);
              A.t[ct][h] = mfma_bf16(xv[h], wlo[ct][ec], A.t[ct][h]);
            }
          }
      } else {
        f32x4 xv[2];
#pragma unroll
        for (int h = 0; h < 2; ++h) xv[h] = phi4(bx, 16 * h + li, 16 * ec + 4 * g);
#pragma unroll
        for (int ct = 0; ct < CT; ++ct)
#pragma unroll
          for (int h = 0; h < 2; ++h)
#pragma unroll
            for (int t = 0; t < 4; ++t) {
              if constexpr (LSE) A.t[ct][h] = mfma_f32(whi[ct][ec][t], xv[h][t], A.t[ct][h]);
              else A.t[ct][h] = mfma_f32(xv[h][t], whi[ct][ec][t], A.t[ct][h]);
            }
      }
    }
    return A;
    }
  };

  // M-GEMM on split bf16 operands (fp32 x): r in three parts (A element j = 4rt + v
  // is data row 16rt + 4g + v), ψ tiles read from the staged split φ rows of
  // buffer bx with the transposing load (rows 4g..4g+3 and 16+4g..16+4g+3, the
  // same order).
  auto mgemm_x3 = [&](const float (&rr)[CT][2][4], int bx) {
    if constexpr (STATS && X3) {
        bf16x8 ra[3][CT];
#pragma unroll
        for (int ct = 0; ct < CT; ++ct) {
          uint32_t q[3][4];
#pragma unroll
          for (int rt = 0; rt < 2; ++rt)
#pragma unroll
            for (int v = 0; v < 4; v += 2)
              split3x2(rr[ct][rt][v], rr[ct][rt][v + 1], q[0][2 * rt + v / 2], q[1][2 * rt + v / 2],
                       q[2][2 * rt + v / 2]);
#pragma unroll
          for (int p = 0; p < 3; ++p) ra[p][ct] = __builtin_bit_cast(bf16x8, make_uint4(q[p][0], q[p][1], q[p][2], q[p][3]));
        }
        // ψ tile jt = 16 consecutive φ columns (diag: x then x², spherical/tied: x) or the
        // augmented columns at EP.
        // Full: ψ = [x | products | 1] from φ = [products | x]; the last tile holds
        // products 128..135 (column groups 0, 1) and the constant chunk at EP
        // (groups 2, 3, whose lane offsets are 8 and 12).
        auto psi_col = [&](int jt) {
          constexpr int XT16 = DP / 16;
          if constexpr (COV == DIAG) return jt < XT16 ? DP + 16 * jt : (jt < 2 * XT16 ? 16 * (jt - XT16) : EP);
          else if constexpr (COV == FULL) return jt == 0 ? S : (jt < JT - 1 ? 16 * (jt - 1) : ((li & 3) < 2 ? S - 8 : EP - 8));
          else return jt < XT16 ? 16 * jt : EP;
        };
        const __bf16* tb = phx + (bx * kBN + 4 * g + (li >> 2)) * EPS + 4 * (li & 3);
#pragma unroll
        for (int jt = 0; jt < JT; ++jt) {
          const int c0 = psi_col(jt);
          bf16x8 bq[3];
#pragma unroll
          for (int p = 0; p < 3; ++p)
            bq[p] = cat_v4s(tr16(tb + p * X3P + c0), tr16(tb + p * X3P + 16 * EPS + c0));
#pragma unroll
          for (int ct = 0; ct < CT; ++ct) {
            acc[ct][jt] = mfma_bf16(ra[0][ct], bq[2], acc[ct][jt]);
            acc[ct][jt] = mfma_bf16(ra[2][ct], bq[0], acc[ct][jt]);
            acc[ct][jt] = mfma_bf16(ra[1][ct], bq[1], acc[ct][jt]);
            acc[ct][jt] = mfma_bf16(ra[0][ct], bq[1], acc[ct][jt]);
            acc[ct][jt] = mfma_bf16(ra[1][ct], bq[0], acc[ct][jt]);
            acc[ct][jt] = mfma_bf16(ra[0][ct], bq[0], acc[ct][jt]);
          }
        }
    }
  };

  auto epilogue = [&](const Acc& A, int bx, int pb, int64_t n0) {
    if constexpr (LSE) {
      // Per data row: wave max (and first argmax) by max-only lane swaps, then one
      // exp per element against that max and a plain sum -- no rescaling.
#pragma unroll
      for (int nt = 0; nt < 2; ++nt) {
        const int r = 16 * nt + li;
        const float rq = rowq_s[bx * kBN + r];
        float l2v[CT][4];
        float m = kLogFloor;
        int idx = 0x7fffffff;
#pragma unroll
        for (int ct = 0; ct < CT; ++ct)
#pragma unroll
          for (int v = 0; v < 4; ++v) {
            const float l2 = logit(cL[ct][v], A.t[ct][nt][v], rq);
            l2v[ct][v] = l2;
            if constexpr (WANT_IDX) {
              if (l2 > m) { m = l2; idx = kbase + 16 * ct + 4 * g + v; }
            } else {
              m = fmaxf(m, l2);
            }
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
          for (int v = 0; v < 4; ++v) s += fast_exp2(l2v[ct][v] - m);
        s = lanes_op<32, false>(lanes_op<16, false>(s));
        // Every lane of the row group holds the same values; all write (no branch).
        const int o = (pb * kBN + r) * 8 + wave;
        red_m[o] = m;
        red_s[o] = s;
        if constexpr (WANT_IDX) red_i[o] = idx;
      }
    } else {
      // Responsibilities for every component tile of this wave.
      float rr[CT][2][4];
      if constexpr (SLSE) {
        // Row r = 16rt + 4g + v: this wave's (max, Σ 2^(l2 - max)) over its
        // components (16 lanes x CT tiles), then the merge over the waves.
        float l2v[CT][2][4];
#pragma unroll
        for (int ct = 0; ct < CT; ++ct)
#pragma unroll
          for (int rt = 0; rt < 2; ++rt)
#pragma unroll
            for (int v = 0; v < 4; ++v)
              l2v[ct][rt][v] = logit(cS[ct], A.t[ct][rt][v], rowq_s[bx * kBN + 16 * rt + 4 * g + v]);
#pragma unroll
        for (int rt = 0; rt < 2; ++rt)
#pragma unroll
          for (int v = 0; v < 4; ++v) {
            float m = kLogFloor;
#pragma unroll
            for (int ct = 0; ct < CT; ++ct) m = fmaxf(m, l2v[ct][rt][v]);
            m = group_max<16>(m);
            float sm = 0.f;
#pragma unroll
            for (int ct = 0; ct < CT; ++ct) sm += fast_exp2(l2v[ct][rt][v] - m);
            sm = group_sum<16>(sm);
            // Every lane of the row group holds the same bits (the reductions pair
            // lanes symmetrically); all write, so no branch splits the eight
            // reductions and the scheduler interleaves their DPP chains (C4 pass
            // 0.55 -> 0.52 ms).  The exchange pass keeps one writer: there the
            // same change measured 4 % slower.
            red_m[(16 * rt + 4 * g + v) * 8 + wave] = m;
            red_s[(16 * rt + 4 * g + v) * 8 + wave] = sm;
          }
        __syncthreads();
        if (lane < kBN) {
          // Two or four waves (small K): unrolled per count (C5 pass 3 % faster);
          // eight: the loop, which measured faster there (C4).
          float M = kLogFloor, S = 0.f;
          if (nw <= 4) {
            merge_waves(nw, red_m + lane * 8, red_s + lane * 8, M, S);
          } else {
            for (int w = 0; w < nw; ++w) M = fmaxf(M, red_m[lane * 8 + w]);
            for (int w = 0; w < nw; ++w) S += red_s[lane * 8 + w] * fast_exp2(red_m[lane * 8 + w] - M);
          }
          const bool valid = n0 + lane < rend;
          const float l = M + __log2f(S);
          lsw[wave * kBN + lane] = valid ? l : INFINITY;
          if (wave == 0 && valid) ll_acc += (double)l;
          // predict_proba with score_samples: the row's log-normaliser is the score
          if constexpr (MODE == MODE_PROBA_LSE)
            if (wave == 0 && valid && a.scores) a.scores[(size_t)b * N + n0 + lane] = l * kLn2;
        }
        // The wave's own LDS writes above are read back by its other lanes below.
        __builtin_amdgcn_fence(__ATOMIC_RELEASE, "wavefront");
        __builtin_amdgcn_fence(__ATOMIC_ACQUIRE, "wavefront");
#pragma unroll
        for (int rt = 0; rt < 2; ++rt) {
          const f32x4 lv = ld16<f32x4>(&lsw[wave * kBN + 16 * rt + 4 * g]);
#pragma unroll
          for (int ct = 0; ct < CT; ++ct)
#pragma unroll
            for (int v = 0; v < 4; ++v) rr[ct][rt][v] = fast_exp2(l2v[ct][rt][v] - lv[v]);
        }
      } else {
#pragma unroll
      for (int ct = 0; ct < CT; ++ct)
#pragma unroll
        for (int rt = 0; rt < 2; ++rt)
#pragma unroll
          for (int v = 0; v < 4; ++v) {
            const int r = BF ? 8 * g + 4 * rt + v : 16 * rt + 4 * g + v;
            const float l2 = logit(cS[ct], A.t[ct][rt][v], rowq_s[bx * kBN + r]);
            if constexpr (MODE == MODE_PROBA) {
              rr[ct][rt][v] = a.raw_logits ? l2 : fast_exp2(l2 - lse_s[bx * kBN + r]);
            } else if constexpr (TOPK) {
              // Only the row's top k (logit descending, then lower index) get mass.
              // (hard: the one component thr_idx, by index, with r = 1 exactly)
              const float t = thr_s[bx * kBN + r];
              const int kk = kbase + 16 * ct + li, ti = thri_s[bx * kBN + r];
              const bool keep = a.hard ? kk == ti : (l2 > t || (l2 == t && kk <= ti));
              rr[ct][rt][v] = keep ? (a.hard ? 1.f : fast_exp2(l2 - lse_s[bx * kBN + r])) : 0.f;
            } else {
              rr[ct][rt][v] = fast_exp2(l2 - lse_s[bx * kBN + r]);
            }
          }
      }
      if constexpr (STATS && X3) {
        mgemm_x3(rr, bx);
      } else if constexpr (STATS) {
        // M-GEMM: each ψ fragment is loaded once and used by every component tile.
        if constexpr (BF) {
          bf16x8 ar[CT];
#pragma unroll
          for (int ct = 0; ct < CT; ++ct)
#pragma unroll
            for (int rt = 0; rt < 2; ++rt)
#pragma unroll
              for (int v = 0; v < 4; ++v) ar[ct][4 * rt + v] = (__bf16)rr[ct][rt][v];
#pragma unroll
          for (int jt = 0; jt < JT; ++jt) {
            const bf16x8 bqv = ld16<bf16x8>(&psiT[pb * JP * QS + (16 * jt + li) * QS + 8 * g]);
#pragma unroll
            for (int ct = 0; ct < CT; ++ct) acc[ct][jt] = mfma_bf16(ar[ct], bqv, acc[ct][jt]);
          }
        } else {
#pragma unroll
          for (int jt = 0; jt < JT; ++jt)
#pragma unroll
            for (int rt = 0; rt < 2; ++rt) {
              float bq[4];
#pragma unroll
              for (int v = 0; v < 4; ++v) bq[v] = psi1(bx, 16 * rt + 4 * g + v, 16 * jt + li);
#pragma unroll
              for (int ct = 0; ct < CT; ++ct)
#pragma unroll
                for (int v = 0; v < 4; ++v) acc[ct][jt] = mfma_f32(rr[ct][rt][v], bq[v], acc[ct][jt]);
            }
        }
      } else {  // MODE_PROBA
#pragma unroll
        for (int ct = 0; ct < CT; ++ct) {
          const int kk = kbase + 16 * ct + li;
          if (kk < K) {
#pragma unroll
            for (int rt = 0; rt < 2; ++rt)
#pragma unroll
              for (int v = 0; v < 4; ++v) {
                const int r = BF ? 8 * g + 4 * rt + v : 16 * rt + 4 * g + v;
                const int64_t n = n0 + r;
                if (n < rend) a.proba[((size_t)b * N + n) * K + kk] = rr[ct][rt][v];
              }
          }
        }
      }
    }
  };

  // ---- main loop: one barrier per block; the loader runs PD blocks ahead ----
  const int64_t nblk = (rend > rbeg) ? (rend - rbeg + kBN - 1) / kBN : 0;
  __syncthreads();  // constant feature rows are in place before any stash or build
  for (int p = 0; p < PD; ++p) {
    if (p < nblk) {
      fetch(rbeg + p * kBN);
      stash(p, rbeg + p * kBN);
    }
  }
  __syncthreads();
  if constexpr (PSI_LDS) {
    if (nblk > 0) build_psi(0, 0);
    __syncthreads();
  }
  Acc cur;
  if constexpr (PIPE) {
    if (nblk > 0) cur = egemm(0);
  }
  if constexpr (XCH) {
    // The a.ktiles workgroups of row slice `slice` (members ktile = 0..ktiles-1,
    // consecutive logical ids, so one XCD when the grid allows) each hold one
    // component tile; per block they swap this workgroup's per-row (max, sum)
    // through global memory, as the cooperative spherical kernel does
    // (em_coop.hip: one 64-bit relaxed agent-scope word (max, sum) per row, bit
    // 31 of the sum half carrying the round parity (j / kRing) & 1, a ring of kRing
    // slots, bounded waits that set *status and stop).  Lag one block: block i's
    // partials are published after its E-GEMM, and block i-1 -- whose logits wait
    // in registers and whose staged rows wait in the extra LDS buffer -- is
    // finished (log-normalisers merged in member order, responsibilities,
    // M-GEMM) after that, when the partners' words for it are a block old.
    // Every wave merges the partials itself, so the only barriers are the two a
    // one-tile pass has.  A slot is rewritten kRing blocks later, after the
    // partners' words of two blocks later have been seen, by which time every
    // wave of every partner has read it.
    const int gm = a.ktiles;
    uint64_t* const gw = a.xch + ((size_t)b * (gridDim.x / gm) + slice) * kRing * gm * kBN;
    float l2p[CT][2][4];
    float Mp = 0.f, Sp = 0.f;     // this workgroup's (max, sum) of the previous block (lanes < 32)
    uint64_t words[kMaxCoopGroup];
    bool dead = false;            // a wait timed out: no further waits
    auto load_words = [&](int64_t j) {
      const uint64_t* src = gw + (j % kRing) * gm * kBN + lane;
#pragma unroll
      for (int p = 0; p < kMaxCoopGroup; ++p)
        words[p] = (p < gm && p != ktile && lane < kBN)
                       ? __hip_atomic_load(src + p * kBN, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT)
                       : 0;
    };
    auto finish = [&](int64_t j, int bxp, int64_t n0p) {
      const bool odd = (j / kRing) & 1;
      // A word is ready when its tag bit matches the round (whatever its data:
      // a NaN or zero sum is passed on, not waited for).
      const uint32_t want = odd ? kTagOdd : 0u;
      auto ready = [&]() {
        uint32_t bad = 0u;
#pragma unroll
        for (int p = 0; p < kMaxCoopGroup; ++p) {
          const uint32_t hi = (uint32_t)(words[p] >> 32);
          bad |= (p < gm && p != ktile && lane < kBN) ? ((hi ^ want) & kTagOdd) : 0u;
        }
        return bad == 0u;
      };
      int spins = 0;
      while (!dead && (a.spin_limit < 0 || __ballot(!ready()) != 0)) {
        if (++spins > a.spin_limit ||
            ((spins & 63) == 0 && __hip_atomic_load(a.status, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT))) {
          dead = true;
          if (lane == 0) __hip_atomic_fetch_or(a.status, 1u, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
          break;
        }
        __builtin_amdgcn_s_sleep(1);
        load_words(j);
      }
      float M = -INFINITY, S = 0.f;
#pragma unroll
      for (int p = 0; p < kMaxCoopGroup; ++p) {
        if (p < gm) {
          const float vm = p == ktile ? Mp : __uint_as_float((uint32_t)words[p]);
          const float vs = p == ktile ? Sp : fabsf(__uint_as_float((uint32_t)(words[p] >> 32)));
          const float Mn = fmaxf(M, vm);
          S = S * fast_exp2(M - Mn) + vs * fast_exp2(vm - Mn);
          M = Mn;
        }
      }
      if (lane < kBN) {
        const bool valid = n0p + lane < rend;
        const float l = M + __log2f(S);
        lsw[wave * kBN + lane] = valid ? l : INFINITY;
        if (ktile == 0 && wave == 0 && valid) ll_acc += (double)l;
      }
      // The wave's own LDS writes above are read back by its other lanes below.
      __builtin_amdgcn_fence(__ATOMIC_RELEASE, "wavefront");
      __builtin_amdgcn_fence(__ATOMIC_ACQUIRE, "wavefront");
      float rr[CT][2][4];
#pragma unroll
      for (int rt = 0; rt < 2; ++rt) {
        const f32x4 lv = ld16<f32x4>(&lsw[wave * kBN + 16 * rt + 4 * g]);
#pragma unroll
        for (int ct = 0; ct < CT; ++ct)
#pragma unroll
          for (int v = 0; v < 4; ++v) rr[ct][rt][v] = fast_exp2(l2p[ct][rt][v] - lv[v]);
      }
      mgemm_x3(rr, bxp);
    };
    for (int64_t ib = 0; ib < nblk; ++ib) {
      const int bx = (int)(ib % NB);
      const int64_t n0 = rbeg + ib * kBN;
      const bool ahead = ib + PD < nblk;
      if (ahead) fetch(n0 + PD * kBN);
      // E-GEMM of block ib: its logits and this wave's (max, Σ 2^(l2 - max)) per row
      const Acc A = egemm(bx);
      float l2c[CT][2][4];
#pragma unroll
      for (int ct = 0; ct < CT; ++ct)
#pragma unroll
        for (int rt = 0; rt < 2; ++rt)
#pragma unroll
          for (int v = 0; v < 4; ++v)
            l2c[ct][rt][v] = logit(cS[ct], A.t[ct][rt][v], rowq_s[bx * kBN + 16 * rt + 4 * g + v]);
#pragma unroll
      for (int rt = 0; rt < 2; ++rt)
#pragma unroll
        for (int v = 0; v < 4; ++v) {
          float m = kLogFloor;
#pragma unroll
          for (int ct = 0; ct < CT; ++ct) m = fmaxf(m, l2c[ct][rt][v]);
          m = group_max<16>(m);
          float sm = 0.f;
#pragma unroll
          for (int ct = 0; ct < CT; ++ct) sm += fast_exp2(l2c[ct][rt][v] - m);
          sm = group_sum<16>(sm);
          if (li == 0) {
            red_m[(16 * rt + 4 * g + v) * 8 + wave] = m;
            red_s[(16 * rt + 4 * g + v) * 8 + wave] = sm;
          }
        }
      // The partners' words of block ib - 1, loaded after the E-GEMM: loaded at
      // the top of the iteration they were often not there yet and the reloads
      // cost more (measured at C3: 3.15 against 3.34 ms per pass).
      if (ib > 0 && !dead) load_words(ib - 1);
      __syncthreads();
      // This workgroup's (max, sum) per row of block ib (lanes < 32), merged by
      // every wave; wave 0 publishes it to the group.
      float M = kLogFloor, S = 0.f;
      if (lane < kBN) {
        for (int w = 0; w < nw; ++w) M = fmaxf(M, red_m[lane * 8 + w]);
        for (int w = 0; w < nw; ++w) S += red_s[lane * 8 + w] * fast_exp2(red_m[lane * 8 + w] - M);
      }
      if (wave == 0 && lane < kBN && gm > 1) {
        const uint32_t tagged = (__float_as_uint(S) & ~kTagOdd) | (((ib / kRing) & 1) ? kTagOdd : 0u);
        const uint64_t word = (uint64_t)__float_as_uint(M) | ((uint64_t)tagged << 32);
        __hip_atomic_store(gw + ((ib % kRing) * gm + ktile) * kBN + lane, word, __ATOMIC_RELAXED,
                           __HIP_MEMORY_SCOPE_AGENT);
      }
      if (ib > 0) finish(ib - 1, (int)((ib - 1) % NB), n0 - kBN);
#pragma unroll
      for (int ct = 0; ct < CT; ++ct)
#pragma unroll
        for (int rt = 0; rt < 2; ++rt)
#pragma unroll
          for (int v = 0; v < 4; ++v) l2p[ct][rt][v] = l2c[ct][rt][v];
      Mp = M;
      Sp = S;
      if (ahead) stash((int)((ib + PD) % NB), n0 + PD * kBN);
      __syncthreads();
    }
    if (nblk > 0) {
      if (!dead) load_words(nblk - 1);
      finish(nblk - 1, (int)((nblk - 1) % NB), rbeg + (nblk - 1) * kBN);
    }
  }
  for (int64_t ib = 0; ib < (XCH ? 0 : nblk); ++ib) {
    const int bx = (int)(ib % NB), pb = (int)(ib & 1);
    const int64_t n0 = rbeg + ib * kBN;
    const bool ahead = ib + PD < nblk;
    if (ahead) fetch(n0 + PD * kBN);
    if constexpr (LSE) {
      if (ib > 0) combine_out(pb ^ 1, n0 - kBN);
    }
    if constexpr (PIPE) {
      // Block ib+1 was staged an iteration ago: its MFMAs run under this block's epilogue.
      // Unconditional (the last iteration reads a stale, in-bounds buffer and
      // discards the result) so the MFMAs share a basic block with the epilogue.
      const Acc nxt = egemm((int)((ib + 1) % NB));
      epilogue(cur, bx, pb, n0);
      cur = nxt;
    } else {
      epilogue(egemm(bx), bx, pb, n0);
    }
    if constexpr (PSI_LDS) {
      if (ib + 1 < nblk) build_psi((int)((ib + 1) % NB), pb ^ 1);
    }
    if constexpr (NB == 1) __syncthreads();   // every wave is done with the only buffer
    if (ahead) stash((int)((ib + PD) % NB), n0 + PD * kBN);
    __syncthreads();
  }
  if constexpr (LSE) {
    if (nblk > 0) combine_out((int)((nblk - 1) & 1), rbeg + (nblk - 1) * kBN);
  }

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
  if constexpr (MODE == MODE_STATS_LSE || XCH) {
    // This workgroup's rows: Σ lse (natural log), one partial per (batch, slice)
    // (exchange pass: from the first member of the group).
    if (wave == 0 && ktile == 0) {
      double t = ll_acc;
#pragma unroll
      for (int off = 32; off >= 1; off /= 2) t += __shfl_xor(t, off);
      if (lane == 0) a.ll_part[(size_t)b * (gridDim.x / a.ktiles) + slice] = t * (double)kLn2;
    }
  }
}

template <int COV, typename XT, int DP>
static int launch_tile_t(int mode, const TileArgs& a, dim3 grid, int nw, hipStream_t s) {
  constexpr int CW = cw_for<COV, DP, sizeof(XT) == 2>();
  const dim3 block(64 * nw);
  switch (mode) {
    case MODE_LSE: em_tile_kernel<COV, XT, DP, CW, MODE_LSE><<<grid, block, 0, s>>>(a); break;
    case MODE_LSE_IDX: em_tile_kernel<COV, XT, DP, CW, MODE_LSE_IDX><<<grid, block, 0, s>>>(a); break;
    case MODE_STATS: em_tile_kernel<COV, XT, DP, CW, MODE_STATS><<<grid, block, 0, s>>>(a); break;
    case MODE_PROBA: em_tile_kernel<COV, XT, DP, CW, MODE_PROBA><<<grid, block, 0, s>>>(a); break;
    case MODE_STATS_TOPK: em_tile_kernel<COV, XT, DP, CW, MODE_STATS_TOPK><<<grid, block, 0, s>>>(a); break;
    case MODE_STATS_LSE: em_tile_kernel<COV, XT, DP, CW, MODE_STATS_LSE><<<grid, block, 0, s>>>(a); break;
    case MODE_PROBA_LSE: em_tile_kernel<COV, XT, DP, CW, MODE_PROBA_LSE><<<grid, block, 0, s>>>(a); break;
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

// ---- exchange pass (MODE_STATS_XCH): grid within the resident capacity, all workgroups co-resident ----

// Every exchange slot starts with the odd round tag, which no round-0 word carries.
__global__ void xch_zero_kernel(uint64_t* w, int64_t n, unsigned* status) {
  const int64_t i = (int64_t)blockIdx.x * blockDim.x + threadIdx.x;
  if (i < n) w[i] = (uint64_t)kTagOdd << 32;
  if (i == 0) *status = 0u;
}

template <int COV, int DP>
static const void* xch_fn() {
  return reinterpret_cast<const void*>(em_tile_kernel<COV, float, DP, cw_for<COV, DP, false>(), MODE_STATS_XCH>);
}

static const void* xch_kernel(int cov, int dp) {
  switch (cov) {
    case SPH:
      return dp == 16 ? xch_fn<SPH, 16>() : dp == 32 ? xch_fn<SPH, 32>() : dp == 64 ? xch_fn<SPH, 64>()
                                          : dp == 128 ? xch_fn<SPH, 128>() : nullptr;
    case DIAG:
      return dp == 16 ? xch_fn<DIAG, 16>() : dp == 32 ? xch_fn<DIAG, 32>() : dp == 64 ? xch_fn<DIAG, 64>() : nullptr;
    case TIED:
      return dp == 16 ? xch_fn<TIED, 16>() : dp == 32 ? xch_fn<TIED, 32>() : dp == 64 ? xch_fn<TIED, 64>() : nullptr;
    default:
      return nullptr;
  }
}

int tile_xch_capacity(int cov, int dp) {
  const void* fn = xch_kernel(cov, dp);
  if (!fn) return 0;
  static std::atomic<int> cache[64][4][8] = {};   // concurrent first calls store the same value
  int ndev = 0, dev = 0;
  if (hipGetDeviceCount(&ndev) != hipSuccess || ndev <= 0 || hipGetDevice(&dev) != hipSuccess || dev >= 64) {
    (void)hipGetLastError();
    return 256;   // no device visible: workspace sizing only
  }
  std::atomic<int>& c = cache[dev][cov & 3][(dp / 16) & 7];
  const int cached = c.load(std::memory_order_relaxed);
  if (cached > 0) return cached;
  int cus = 0, per = 0;
  if (hipDeviceGetAttribute(&cus, hipDeviceAttributeMultiprocessorCount, dev) != hipSuccess ||
      hipOccupancyMaxActiveBlocksPerMultiprocessor(&per, fn, 64 * 8, 0) != hipSuccess || cus <= 0 || per <= 0) {
    (void)hipGetLastError();
    return 0;
  }
  c.store(cus * per, std::memory_order_relaxed);
  return cus * per;
}

int launch_tile_xch(int cov, int dp, const TileArgs& a, dim3 grid, int64_t nwords, hipStream_t s) {
  const void* fn = xch_kernel(cov, dp);
  if (!fn) return -1;
  xch_zero_kernel<<<(unsigned)((nwords + 255) / 256 + 1), 256, 0, s>>>(a.xch, nwords, a.status);
  // At most the resident capacity, as a plain launch (em_coop.hip): the bounded
  // waits guard against members that are not co-resident.
  if ((int64_t)grid.x * grid.y * grid.z > tile_xch_capacity(cov, dp)) return -1;
  TileArgs args = a;
  void* params[] = {&args};
  if (hipLaunchKernel(fn, grid, dim3(64 * 8), params, 0, s) != hipSuccess) {
    (void)hipGetLastError();
    return -2;
  }
  return 0;
}

int launch_tile(int cov, int bf, int dp, int mode, const TileArgs& a, dim3 grid, int nw, hipStream_t s) {
  switch (cov) {
    case SPH:
      return bf ? -1 : launch_tile_dp<SPH, float>(dp, mode, a, grid, nw, s);  // bf16: em_sph_bf16.hip
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
