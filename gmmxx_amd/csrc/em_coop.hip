// Single-pass spherical bf16 EM tile for many components at D = 128.
//
// The two-pass tile design (em_sph_bf16.hip) computes every logit twice: once
// for the row log-normalisers and once more for the responsibilities, because
// the component tiles of one row live in different workgroups.  Here the
// workgroups that cover the component tiles of the same rows form a GROUP
// (G = ceil(K / 256) workgroups, 8 waves x 32 components each) and swap each
// row block's per-row (max, scaled sum) partials through global memory, so the
// E-GEMM runs once per (row, component) and its exponentials are reused:
//
//   block i:    E-GEMM (logits l2, log2 units, as in em_sph_bf16.hip)
//               m_w = wave row max, e = 2^(l2 - m_w) (kept in LDS as bf16), s_w = Σ e
//               workgroup partials (M, S) per row -> published to the group
//   block i-2:  lse2 = merge of the group's partials (same order in every
//               member, so all members use bit-identical log-normalisers)
//               r = e · 2^(m_w - lse2), staged row-major in LDS and read back
//               with the transposing load as the A operand of the M-GEMM
//               acc += rᵀ·ψ (ψ = the staged row [x | augmented columns]).
//
// The two-block lag hides the exchange: wave 1 publishes block i-1 at the top
// of iteration i, and wave 0 collects the group's partials of block i-1 (its own
// workgroup's word included) at its end, after a whole block of MFMA work.  The
// two roles sit on different waves (and SIMDs) because every wave waits at the
// block's barrier for the slowest one: split, they cost the larger of the two
// instead of their sum (measured 4.57 -> 4.15 ms per C2 pass).  Members of one
// group must run at the same
// time, so the kernel launches cooperatively (all workgroups co-resident); every
// wait is bounded (spin limit), and a wait that times out sets *status and
// stops waiting, so the kernel always drains.  Used for 2 <= G <= 4: with one
// member the two-pass kernels are faster, and eight members wait on each other
// too often (both measured).  Groups are placed on one XCD
// (workgroup ids congruent mod 8) so the exchange stays in that XCD's L2.
// (Agent-scope release/acquire fences instead write back and invalidate the
// L2 at every block: the same kernel with them measured 13.4 ms per C2 pass.)
//
// Exchange protocol (no fences): the pair of block j (j = blocks the group has
// exchanged before) goes to slot j % kRing as one 64-bit relaxed agent-scope
// atomic store of (M, ±S), the sign of S carrying the round parity
// (j / kRing) & 1 (S > 0 always; the launcher zeroes the slots, and a zero S
// matches neither sign).  A reader polls each partner's 64-bit word with
// relaxed agent-scope atomic loads until the sign matches the expected round,
// so every datum is checked on its own and no ordering between addresses is
// needed.  A slot is rewritten only after every partner has read it: a member
// publishes block j after it has received every partner's block j - 1, which
// they publish after finishing their reads of block j - 2, so a ring of two
// slots would do; four are used.  A slot therefore holds block j or block
// j - kRing, which the parity tag tells apart.

#include <type_traits>

#include "common.hpp"
#include "engine.hpp"

namespace gx {

namespace {

constexpr int kAug = 32;           // augmented k-chunk width (bf16 columns)
constexpr float kHuge = 1e30f;     // "minus infinity" that stays finite through MFMA
constexpr int kNW = 8;             // waves per workgroup
constexpr int kCW = 32;            // components per wave
constexpr int kCT = 2;             // 16-wide component tiles per wave
constexpr int kNB = 5;             // staged row blocks: i-2 .. i+2
constexpr int kRS = 48;            // r row stride (bf16): 32 components + padding

typedef short v4s __attribute__((ext_vector_type(4)));
typedef __bf16 bf16x2 __attribute__((ext_vector_type(2)));
typedef float f32x2 __attribute__((ext_vector_type(2)));

template <typename T>
__device__ __forceinline__ T ld16(const void* p) { return *reinterpret_cast<const T*>(p); }

template <int CTRL>
__device__ __forceinline__ float dpp(float v) {
  return __int_as_float(__builtin_amdgcn_update_dpp(0, __float_as_int(v), CTRL, 0xF, 0xF, false));
}

// Sum over groups of G consecutive lanes (G <= 16), result in every lane.
template <int G>
__device__ __forceinline__ float group_sum(float v) {
  if constexpr (G >= 2) v += dpp<0xB1>(v);    // lane ^ 1
  if constexpr (G >= 4) v += dpp<0x4E>(v);    // lane ^ 2
  if constexpr (G >= 8) v += dpp<0x141>(v);   // row_half_mirror
  if constexpr (G >= 16) v += dpp<0x140>(v);  // row_mirror
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

__device__ __forceinline__ void split3(float v, __bf16& h, __bf16& m, __bf16& l) {
  h = (__bf16)v;
  const float r = v - (float)h;
  m = (__bf16)r;
  l = (__bf16)(r - (float)m);
}

__device__ __forceinline__ uint32_t pack2(__bf16 a, __bf16 b) {
  return (uint32_t)__builtin_bit_cast(uint16_t, a) | ((uint32_t)__builtin_bit_cast(uint16_t, b) << 16);
}

// Two floats rounded to bf16 (nearest even) in one dword, a in the low half.
__device__ __forceinline__ uint32_t cvt2(float a, float b) {
  return __builtin_bit_cast(uint32_t, __builtin_convertvector(f32x2{a, b}, bf16x2));
}

// Transposing LDS read: in each 16-lane group, lane L supplies the address of
// an 8-byte chunk; lane i receives word (i % 4) of the chunks of lanes 4j + i/4.
__device__ __forceinline__ v4s tr16(const __bf16* p) {
  return __builtin_amdgcn_ds_read_tr16_b64_v4i16((__attribute__((address_space(3))) v4s*)p);
}

__device__ __forceinline__ bf16x8 cat(v4s lo, v4s hi) {
  return __builtin_bit_cast(bf16x8, __builtin_shufflevector(lo, hi, 0, 1, 2, 3, 4, 5, 6, 7));
}

// r rows: the 4-element column chunk is XOR-swizzled by (row / 4) % 4, so that
// 16 lanes writing one chunk of consecutive rows, and the transposing reads of
// 4 rows x 4 chunks, touch distinct bank pairs.
__device__ __forceinline__ int rswz(int row, int col) { return col ^ (((row >> 2) & 3) << 2); }

__global__ void coop_zero_kernel(unsigned* p, int n, unsigned* status) {
  const int i = blockIdx.x * blockDim.x + threadIdx.x;
  if (i < n) p[i] = 0u;
  if (i == n) *status = 0u;
}

}  // namespace

// KG: largest group size the instance handles (G <= KG); the partners' words of
// a block are loaded together into KG registers.
template <int DP, int KG>
__global__ __launch_bounds__(64 * kNW) void sph_bf16_coop_kernel(CoopArgs a) {
  constexpr int ECH = DP / 32;                   // x chunks of the E-GEMM
  constexpr int XS = 176;                        // staged row stride (bf16), as em_sph_bf16.hip at D = 128
  static_assert(DP + kAug <= XS, "row does not fit the staging stride");
  constexpr int JT = DP / 16 + 1;                // ψ = [x | augmented columns 0..15]
  constexpr int JP = 16 * JT;
  constexpr int CPR = DP / 8;                    // 16-byte chunks per row
  constexpr int NCH = kBN * CPR;                 // chunks per row block
  constexpr int NTHR = 64 * kNW;
  constexpr int PF = (NCH + NTHR - 1) / NTHR;
  constexpr int RR = kBN + 1;                    // red_* stride per wave
  static_assert(NCH % 64 == 0, "row block must split into whole waves of chunks");

  __shared__ __align__(16) __bf16 xs[kNB * kBN * XS];
  __shared__ __align__(16) __bf16 rs[kNW * kBN * kRS];
  __shared__ float red_m[2 * kNW * RR];
  __shared__ float red_s[2 * kNW * RR];
  __shared__ float lse_s[2 * kBN];
  // e = 2^(l2 - m_w) of the two blocks in flight, per wave and block parity, in
  // the accumulator layout (four bf16 per lane and (ct, row tile)); kept in LDS,
  // which leaves the registers to the W operands and the statistics.  e is
  // rounded to bf16 here and r = e·2^(m_w - lse2) again before the M-GEMM (r is a
  // bf16 MFMA operand in any case): half the LDS bytes of fp32 e, measured 3 %
  // faster at K = 1024, with the sums and the log-normalisers still from fp32 e.
  __shared__ uint2 es[kNW * 2 * kCT * 2 * 64];

  const int tid = threadIdx.x;
  const int wave = tid / 64, lane = tid % 64;
  const int g = lane / 16, li = lane % 16;
  const int64_t N = a.N;
  const int K = a.K, G = a.G;

  // Group and member: groups on one XCD (ids congruent mod 8) when NG % 8 == 0.
  const int id = blockIdx.x;
  int grp, mem;
  if (a.NG % 8 == 0) {
    const int j = id / 8;
    grp = id % 8 + 8 * (j / G);
    mem = j % G;
  } else {
    grp = id / G;
    mem = id % G;
  }
  grp = __builtin_amdgcn_readfirstlane(grp);   // uniform: keep the exchange bases in SGPRs
  mem = __builtin_amdgcn_readfirstlane(mem);
  const int kbase = mem * (kNW * kCW) + __builtin_amdgcn_readfirstlane(wave) * kCW;
  uint64_t* const gxch = a.xch + (size_t)grp * kRing * G * kBN;

  // Constant augmented columns 8..31 of every staged row: [1 0 0 ...]; the
  // e slots start at zero, so no LDS word is read before it is written.
  for (int i = tid; i < kNB * kBN * 3; i += NTHR) {
    const int row = i / 3, ch = 1 + i % 3;
    const uint4 w = make_uint4(ch == 1 ? pack2((__bf16)1.f, (__bf16)0.f) : 0u, 0u, 0u, 0u);
    *reinterpret_cast<uint4*>(xs + row * XS + DP + 8 * ch) = w;
  }
  for (int i = tid; i < kNW * 2 * kCT * 2 * 64; i += NTHR) es[i] = make_uint2(0u, 0u);

  bf16x8 whi[kCT][ECH], wlo[kCT][ECH], waug[kCT];
  f32x4 acc[kCT][JT];
  float mw[2][2];          // wave row maxima of the two blocks in flight: [block parity][row tile]
  unsigned seq = 0;        // blocks this group has exchanged before the current item
  bool dead = false;       // wave 0: a wait timed out; no further waits

  const int items = a.B * a.spb;
  for (int item = grp; item < items; item += a.NG) {
    const int b = item / a.spb, sl = item % a.spb;
    const int64_t rbeg = (int64_t)sl * a.rows_per_item;
    const int64_t rend = (rbeg + a.rows_per_item < N) ? rbeg + a.rows_per_item : N;
    const int nblk = (rend > rbeg) ? (int)((rend - rbeg + kBN - 1) / kBN) : 0;

    // ---- resident component operands (A side of the E-GEMM): lane (li, g) holds
    // component kbase + 16ct + li, k-group g; padding components get C = -1e30. ----
#pragma unroll
    for (int ct = 0; ct < kCT; ++ct) {
      const int kk = kbase + 16 * ct + li;
      if (kk < K) {
        const size_t bk = (size_t)b * K + kk;
#pragma unroll
        for (int ec = 0; ec < ECH; ++ec) {
          whi[ct][ec] = ld16<bf16x8>(reinterpret_cast<const __bf16*>(a.w_hi) + bk * DP + 32 * ec + 8 * g);
          wlo[ct][ec] = ld16<bf16x8>(reinterpret_cast<const __bf16*>(a.w_lo) + bk * DP + 32 * ec + 8 * g);
        }
        waug[ct] = ld16<bf16x8>(reinterpret_cast<const __bf16*>(a.w_aug) + bk * kAug + 8 * g);
      } else {
#pragma unroll
        for (int s = 0; s < 8; ++s) {
#pragma unroll
          for (int ec = 0; ec < ECH; ++ec) { whi[ct][ec][s] = (__bf16)0.f; wlo[ct][ec][s] = (__bf16)0.f; }
          waug[ct][s] = (__bf16)((8 * g + s) == 6 ? -kHuge : 0.f);
        }
      }
#pragma unroll
      for (int jt = 0; jt < JT; ++jt) acc[ct][jt] = f32x4{0.f, 0.f, 0.f, 0.f};
    }
    double ll = 0.0;

    // x rows of this item, addressed with 32-bit offsets from a uniform base (the
    // launcher keeps an item under 2^31 bytes).  Rows past the item end read the
    // last valid row (in bounds, no branch) and are zeroed.
    const __bf16* xi = reinterpret_cast<const __bf16*>(a.x) + ((size_t)b * N + rbeg) * DP;
    const int nrows = (int)(rend - rbeg);
    uint4 pf[PF];
    auto load_chunk = [&](int c, int r0) -> uint4 {
      const int r = r0 + c / CPR, cc = (c % CPR) * 8;
      const bool valid = r < nrows;
      const uint4 v = *reinterpret_cast<const uint4*>(xi + (valid ? r : nrows - 1) * DP + cc);
      return valid ? v : make_uint4(0, 0, 0, 0);
    };
    auto fetch = [&](int r0) {
#pragma unroll
      for (int i = 0; i < PF; ++i) {
        const int c = tid + i * NTHR;
        if (NCH % NTHR == 0 || c < NCH) pf[i] = load_chunk(c, r0);
      }
    };
    // Stages the prefetched block into buffer `buf`: x, and columns 0..7 of the
    // augmented chunk [q_h q_m q_l q_h q_m q_h 1 1] with q = ‖x‖².
    auto stash = [&](int buf) {
#pragma unroll
      for (int i = 0; i < PF; ++i) {
        const int c = tid + i * NTHR;
        if (NCH % NTHR == 0 || c < NCH) {
          const int r = c / CPR, cc = c % CPR;
          const uint4 raw = pf[i];
          __bf16* row = xs + buf * kBN * XS + r * XS;
          *reinterpret_cast<uint4*>(row + 8 * cc) = raw;
          const uint32_t w4[4] = {raw.x, raw.y, raw.z, raw.w};
          float q = 0.f;
#pragma unroll
          for (int j = 0; j < 4; ++j) {
            const bf16x2 p = __builtin_bit_cast(bf16x2, w4[j]);
            q = __builtin_amdgcn_fdot2_f32_bf16(p, p, q, false);
          }
          q = group_sum<CPR>(q);
          if (cc == 0) {
            __bf16 h, m, l;
            split3(q, h, m, l);
            *reinterpret_cast<uint4*>(row + DP) =
                make_uint4(pack2(h, m), pack2(l, h), pack2(m, h), pack2((__bf16)1.f, (__bf16)1.f));
          }
        }
      }
    };

    // Responsibilities of block i-2 (parity pb, first row rf): r = e · 2^(m_w - lse2)
    // with e read back (bf16) from this wave's LDS slot, rounded to bf16 and staged
    // row-major for the transposing reads of the M-GEMM.
    auto prep_r = [&](auto PB_, int rf, int nr) {
      constexpr int pb = decltype(PB_)::value;
      float f[2];
#pragma unroll
      for (int h = 0; h < 2; ++h) {
        const int r = 16 * h + li;
        const float l2 = lse_s[pb * kBN + r];   // read unconditionally: no branch around the LDS load
        f[h] = (rf + r < nr) ? fast_exp2(mw[pb][h] - l2) : 0.f;
      }
      __bf16* rw = rs + wave * kBN * kRS;
      const uint2* ew = es + ((wave * 2 + pb) * kCT * 2) * 64 + lane;
#pragma unroll
      for (int ct = 0; ct < kCT; ++ct)
#pragma unroll
        for (int h = 0; h < 2; ++h) {
          const uint2 q = ew[(ct * 2 + h) * 64];
          const f32x2 e01 = __builtin_convertvector(__builtin_bit_cast(bf16x2, q.x), f32x2);
          const f32x2 e23 = __builtin_convertvector(__builtin_bit_cast(bf16x2, q.y), f32x2);
          const f32x4 e = f32x4{e01[0], e01[1], e23[0], e23[1]};
          const int r = 16 * h + li;
          const uint2 pk = make_uint2(cvt2(e[0] * f[h], e[1] * f[h]), cvt2(e[2] * f[h], e[3] * f[h]));
          *reinterpret_cast<uint2*>(rw + r * kRS + rswz(r, 16 * ct + 4 * g)) = pk;
        }
    };
    // M-GEMM of a staged block: A = r[component 16ct + li][rows 4g..4g+3, 16+4g..16+4g+3],
    // B = ψ of the same rows, feature 16jt + li (the k order of both operands matches).
    auto mgemm = [&](int bx) {
      const __bf16* rw = rs + wave * kBN * kRS;
      bf16x8 ar[kCT];
      const int tr = 4 * g + (li >> 2), c0 = 4 * (li & 3);
#pragma unroll
      for (int ct = 0; ct < kCT; ++ct)
        ar[ct] = cat(tr16(rw + tr * kRS + rswz(tr, 16 * ct + c0)),
                     tr16(rw + (tr + 16) * kRS + rswz(tr + 16, 16 * ct + c0)));
      const __bf16* xr = xs + bx * kBN * XS + tr * XS + c0;
      // B operands are read one feature tile ahead of their MFMAs, so the LDS
      // latency of tile jt + 1 hides behind the MFMAs of tile jt.
      bf16x8 bn = cat(tr16(xr), tr16(xr + 16 * XS));
#pragma unroll
      for (int jt = 0; jt < JT; ++jt) {
        const bf16x8 bq = bn;
        if (jt + 1 < JT) bn = cat(tr16(xr + 16 * (jt + 1)), tr16(xr + 16 * XS + 16 * (jt + 1)));
#pragma unroll
        for (int ct = 0; ct < kCT; ++ct) acc[ct][jt] = mfma_bf16(ar[ct], bq, acc[ct][jt]);
      }
    };
    // E-GEMM C = W·φᵀ of a staged block: lane (li, g) gets components 16ct + 4g + v
    // of row 16h + li.
    auto egemm = [&](int bx, f32x4 (&T)[kCT][2]) {
      const __bf16* xr = xs + bx * kBN * XS + li * XS + 8 * g;
#pragma unroll
      for (int h = 0; h < 2; ++h) {
        const bf16x8 xa = ld16<bf16x8>(xr + 16 * h * XS + DP);
#pragma unroll
        for (int ct = 0; ct < kCT; ++ct) T[ct][h] = mfma_bf16(waug[ct], xa, f32x4{0.f, 0.f, 0.f, 0.f});
      }
#pragma unroll
      for (int ec = 0; ec < ECH; ++ec) {
        bf16x8 xv[2];
#pragma unroll
        for (int h = 0; h < 2; ++h) xv[h] = ld16<bf16x8>(xr + 16 * h * XS + 32 * ec);
#pragma unroll
        for (int ct = 0; ct < kCT; ++ct)
#pragma unroll
          for (int h = 0; h < 2; ++h) T[ct][h] = mfma_bf16(whi[ct][ec], xv[h], T[ct][h]);
#pragma unroll
        for (int ct = 0; ct < kCT; ++ct)
#pragma unroll
          for (int h = 0; h < 2; ++h) T[ct][h] = mfma_bf16(wlo[ct][ec], xv[h], T[ct][h]);
      }
    };
    // Wave row maxima m_w, e = 2^(l2 - m_w) (kept in this wave's LDS slot of the
    // block parity) and the wave's row sums for the workgroup combine.
    auto lse_epilogue = [&](const f32x4 (&T)[kCT][2], auto PB_) {
      constexpr int pb = decltype(PB_)::value;
      uint2* ew = es + ((wave * 2 + pb) * kCT * 2) * 64 + lane;
#pragma unroll
      for (int h = 0; h < 2; ++h) {
        float m = T[0][h][0];
#pragma unroll
        for (int ct = 0; ct < kCT; ++ct)
#pragma unroll
          for (int v = 0; v < 4; ++v) m = fmaxf(m, T[ct][h][v]);
        m = lanes_op<32, true>(lanes_op<16, true>(m));
        float sum = 0.f;
#pragma unroll
        for (int ct = 0; ct < kCT; ++ct) {
          f32x4 e;
#pragma unroll
          for (int v = 0; v < 4; ++v) e[v] = fast_exp2(T[ct][h][v] - m);
          sum += (e[0] + e[1]) + (e[2] + e[3]);
          ew[(ct * 2 + h) * 64] = make_uint2(cvt2(e[0], e[1]), cvt2(e[2], e[3]));
        }
        sum = lanes_op<32, false>(lanes_op<16, false>(sum));
        mw[pb][h] = m;
        // The four lanes of a row hold the same values: all of them store (no branch).
        red_m[(pb * kNW + wave) * RR + 16 * h + li] = m;
        red_s[(pb * kNW + wave) * RR + 16 * h + li] = sum;
      }
    };
    if (nblk > 0) { fetch(0); stash(0); }
    if (nblk > 1) { fetch(kBN); stash(1); }
    __syncthreads();

    // Iteration i of the block pipeline.  FIN: block i-2 is finished (i >= 2);
    // EGM: block i is computed (i < nblk); PB = i & 1, the LDS/register slot
    // parity of blocks i and i-2.  The flags are compile-time, so the steady
    // state (both) is one basic block per half that the scheduler interleaves.
    auto step = [&](auto FIN_, auto EGM_, auto PB_, int i) {
      constexpr bool FIN = decltype(FIN_)::value, EGM = decltype(EGM_)::value;
      constexpr int PB = decltype(PB_)::value;
      const int r0 = i * kBN;                     // first row of block i in the item
      const bool ahead = i + 2 < nblk;
      if (ahead) fetch(r0 + 2 * kBN);
      const bool xchg = wave == 0 && i >= 1 && i <= nblk;   // wave 0 collects block i-1
      const bool pubw = wave == 1 && i >= 1 && i <= nblk;   // wave 1 publishes block i-1

      // ---- wave 1: this workgroup's partials of block i-1, published to the group ----
      float ownM = 0.f, ownS = 0.f;
      if (pubw) {
        if (lane < kBN) {
          constexpr int qb = PB ^ 1;              // parity of block i-1
          float M = red_m[(qb * kNW) * RR + lane];
#pragma unroll
          for (int w = 1; w < kNW; ++w) M = fmaxf(M, red_m[(qb * kNW + w) * RR + lane]);
          float S = 0.f;
#pragma unroll
          for (int w = 0; w < kNW; ++w)
            S += red_s[(qb * kNW + w) * RR + lane] * fast_exp2(red_m[(qb * kNW + w) * RR + lane] - M);
          ownM = M;
          ownS = S;
          if (G > 1) {
            const unsigned j = seq + i - 1;
            const float tagged = ((j / kRing) & 1) ? -S : S;
            const uint64_t word = (uint64_t)__float_as_uint(M) | ((uint64_t)__float_as_uint(tagged) << 32);
            __hip_atomic_store(gxch + ((j % kRing) * G + mem) * kBN + lane, word, __ATOMIC_RELAXED,
                               __HIP_MEMORY_SCOPE_AGENT);
          }
        }
      }

      // ---- responsibilities of block i-2 with the E-GEMM of block i ----
      f32x4 T[kCT][2];
      if constexpr (FIN) prep_r(PB_, r0 - 2 * kBN, nrows);
      if constexpr (EGM) egemm(i % kNB, T);

      // ---- wave 0: the group's words of block i-1 (published at the top of this
      // iteration; this workgroup's own included), loaded now and checked after
      // the second half ----
      uint64_t words[KG];
      const unsigned jx = seq + i - 1;
      const uint64_t* src = gxch + (jx % kRing) * G * kBN + lane;
      auto load_words = [&]() {
#pragma unroll
        for (int p = 0; p < KG; ++p)
          words[p] = (p < G && lane < kBN)
                         ? __hip_atomic_load(src + p * kBN, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT)
                         : 0;
      };
      if (KG > 1 && xchg && !dead) load_words();

      // ---- M-GEMM of block i-2 with the E epilogue of block i ----
      if constexpr (FIN) {
        // The staging writes of prep_r and the transposing reads below are LDS
        // operations of this wave only, executed in order; keep the compiler
        // from reordering them.
        __builtin_amdgcn_fence(__ATOMIC_RELEASE, "wavefront");
        __builtin_amdgcn_fence(__ATOMIC_ACQUIRE, "wavefront");
        mgemm((i - 2) % kNB);
      }
      if constexpr (EGM) lse_epilogue(T, PB_);
      if constexpr (FIN) {
        __builtin_amdgcn_fence(__ATOMIC_RELEASE, "wavefront");
        __builtin_amdgcn_fence(__ATOMIC_ACQUIRE, "wavefront");
      }

      // ---- wave 0: the group's log-normalisers of block i-1 ----
      if (xchg) {
        float M = ownM, S = ownS;
        if (KG > 1 && G > 1) {
          const bool odd = (jx / kRing) & 1;
          auto ready = [&]() {
            bool ok = true;
#pragma unroll
            for (int p = 0; p < KG; ++p) {
              const float t = __uint_as_float((uint32_t)(words[p] >> 32));
              if (p < G && lane < kBN) ok = ok && (odd ? t < 0.f : t > 0.f);
            }
            return ok;
          };
          // A negative spin limit gives up at the first wait (the host's way to
          // exercise the timeout path without a stalled partner).
          int spins = 0;
          while (!dead && (a.spin_limit < 0 || __ballot(!ready()) != 0)) {
            if (++spins > a.spin_limit ||
                ((spins & 63) == 0 && __hip_atomic_load(a.status, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT))) {
              dead = true;
              if (lane == 0) __hip_atomic_fetch_or(a.status, 1u, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
              break;
            }
            __builtin_amdgcn_s_sleep(1);
            load_words();
          }
          // Every member merges the same words in member order: the same bits.
          M = -INFINITY;
#pragma unroll
          for (int p = 0; p < KG; ++p)
            if (p < G) M = fmaxf(M, __uint_as_float((uint32_t)words[p]));
          S = 0.f;
#pragma unroll
          for (int p = 0; p < KG; ++p)
            if (p < G)
              S += fabsf(__uint_as_float((uint32_t)(words[p] >> 32))) *
                   fast_exp2(__uint_as_float((uint32_t)words[p]) - M);
        }
        if (lane < kBN) {
          const float l2 = M + __log2f(S);
          lse_s[(PB ^ 1) * kBN + lane] = l2;
          if (mem == 0 && r0 - kBN + lane < nrows) ll += (double)l2;
        }
      }

      if (ahead) stash((i + 2) % kNB);
      __syncthreads();
    };
    using T_ = std::integral_constant<bool, true>;
    using F_ = std::integral_constant<bool, false>;
    using P0 = std::integral_constant<int, 0>;
    using P1 = std::integral_constant<int, 1>;
    step(F_{}, T_{}, P0{}, 0);                                  // nblk >= 1
    if (nblk > 1) step(F_{}, T_{}, P1{}, 1);
    else step(F_{}, F_{}, P1{}, 1);
    int i = 2;
    for (; i + 1 < nblk; i += 2) {
      step(T_{}, T_{}, P0{}, i);
      step(T_{}, T_{}, P1{}, i + 1);
    }
    if (i < nblk) { step(T_{}, T_{}, P0{}, i); ++i; }
    // drain: the last two blocks are finished (i = nblk, nblk + 1); an item of
    // one block has only block 0 left (i = 2), and block 1 was never staged.
    if (nblk == 1) step(T_{}, F_{}, P0{}, 2);
    else if (i & 1) { step(T_{}, F_{}, P1{}, i); step(T_{}, F_{}, P0{}, i + 1); }
    else { step(T_{}, F_{}, P0{}, i); step(T_{}, F_{}, P1{}, i + 1); }
    seq += (unsigned)nblk;

    // ---- the item's partial statistics (lane (li, g): component 4g + v of the
    // tile, feature 16jt + li) and log-likelihood (natural log) ----
#pragma unroll
    for (int ct = 0; ct < kCT; ++ct)
#pragma unroll
      for (int v = 0; v < 4; ++v) {
        const int kk = kbase + 16 * ct + 4 * g + v;
        if (kk < K) {
          float* dst = a.part_stats + (((size_t)sl * a.B + b) * K + kk) * JP;
#pragma unroll
          for (int jt = 0; jt < JT; ++jt) dst[16 * jt + li] = acc[ct][jt][v];
        }
      }
    if (mem == 0 && wave == 0) {
      for (int off = 32; off >= 1; off /= 2) ll += __shfl_xor(ll, off);
      if (lane == 0) a.ll_part[(size_t)b * a.spb + sl] = ll * (double)kLn2;
    }
  }
}

int coop_capacity() {
  // Resident workgroups of the kernel on the current device (cached per device);
  // 256 when no device is visible (workspace sizing on a machine without a GPU).
  static int cache[64] = {0};
  int ndev = 0, dev = 0;
  if (hipGetDeviceCount(&ndev) != hipSuccess || ndev <= 0 || hipGetDevice(&dev) != hipSuccess || dev >= 64) {
    (void)hipGetLastError();
    return 256;
  }
  if (cache[dev] > 0) return cache[dev];
  int cus = 0, per = 0;
  if (hipDeviceGetAttribute(&cus, hipDeviceAttributeMultiprocessorCount, dev) != hipSuccess ||
      hipOccupancyMaxActiveBlocksPerMultiprocessor(&per, sph_bf16_coop_kernel<128, 4>, 64 * kNW, 0) != hipSuccess ||
      cus <= 0 || per <= 0) {
    (void)hipGetLastError();
    return 256;
  }
  cache[dev] = cus * per;
  return cache[dev];
}

int launch_sph_bf16_coop(int dp, const CoopArgs& a, hipStream_t s) {
  if (dp != 128 || a.G < 2 || a.G > kMaxCoopGroup) return -1;
  const int grid = a.NG * a.G;
  // The exchange slots (64-bit words) and the status word start at zero.
  const int nwords = a.NG * kRing * a.G * kBN * 2;
  coop_zero_kernel<<<(nwords + 1 + 255) / 256, 256, 0, s>>>(reinterpret_cast<unsigned*>(a.xch), nwords, a.status);
  const void* fn = a.G <= 2 ? reinterpret_cast<const void*>(sph_bf16_coop_kernel<128, 2>)
                            : reinterpret_cast<const void*>(sph_bf16_coop_kernel<128, 4>);
  CoopArgs args = a;
  void* params[] = {&args};
  const hipError_t e = hipLaunchCooperativeKernel(fn, dim3(grid), dim3(64 * kNW), params, 0, s);
  if (e != hipSuccess) {
    (void)hipGetLastError();
    return -2;
  }
  return 0;
}

}  // namespace gx
