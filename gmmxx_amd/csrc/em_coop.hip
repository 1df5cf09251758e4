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
// Both GEMMs run on the 32x32x16 bf16 MFMA (as em_fused.hip): a wave's E-GEMM
// output is one 32-component x 32-row tile whose lane l holds 16 components of
// row l % 32 (lane l ^ 32 the other 16), so the row maxima and sums are in-lane
// work plus one lane swap (measured 2 % faster per C2 pass than 16x16x32 tiles,
// whose rows spread over four lanes).
//
//   block i:    E-GEMM: logits l2 (log2 units) = (log2(e)/σ²)·(x·μ) + A·‖x‖² + C,
//               the exact product of bf16 x and bf16 means on MFMA, scaled in
//               fp32 (the two-pass kernels split -2·ca·μ into bf16 hi + lo
//               instead: twice the MFMA work), the rest from the augmented chunk
//               m_w = wave row max, e = 2^(l2 - m_w) (kept in fp32 registers), s_w = Σ e
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
// group must run at the same time, so the grid is at most the kernel's resident
// capacity (all workgroups dispatched at once on an idle device; a plain launch,
// not the cooperative-launch API); every wait is bounded (spin limit), and a
// wait that times out sets *status and stops waiting, so the kernel always
// drains.  Used for 2 <= G <= 4: with one
// member the two-pass kernels are faster, and eight members wait on each other
// too often (both measured).  Groups are placed on one XCD
// (workgroup ids congruent mod 8) so the exchange stays in that XCD's L2.
// (Agent-scope release/acquire fences instead write back and invalidate the
// L2 at every block: the same kernel with them measured 13.4 ms per C2 pass.)
//
// Exchange protocol (no fences): the pair of block j (j = blocks the group has
// exchanged before) goes to slot j % kRing as one 64-bit relaxed agent-scope
// atomic store of (M, S) with bit 31 of the S half replaced by the round parity
// (j / kRing) & 1 (S >= 0, so the bit carries no data, and the tag is the same
// for a NaN, infinite or zero S: a non-finite row propagates into the
// parameters as in the reference instead of stalling the exchange).  The
// launcher fills every slot with the odd tag, which no round-0 word carries.
// A reader polls each partner's 64-bit word with relaxed agent-scope atomic
// loads until the tag matches the expected round, so every datum is checked
// on its own and no ordering between addresses is needed.  A slot is rewritten only after every partner has read it: a member
// publishes block j after it has received every partner's block j - 1, which
// they publish after finishing their reads of block j - 2, so a ring of two
// slots would do; four are used.  A slot therefore holds block j or block
// j - kRing, which the parity tag tells apart.

#include <atomic>
#include <type_traits>

#include "common.hpp"
#include "engine.hpp"

namespace gx {

namespace {

constexpr int kAug = 32;           // augmented k-chunk width (bf16 columns)
constexpr float kHuge = 1e30f;     // "minus infinity" that stays finite through MFMA
constexpr int kNW = 8;             // waves per workgroup
constexpr int kCW = 32;            // components per wave
constexpr int kNB = 5;             // staged row blocks: i-2 .. i+2
constexpr int kRS = 48;            // r row stride (bf16): 32 components + padding

typedef short v4s __attribute__((ext_vector_type(4)));
typedef __bf16 bf16x2 __attribute__((ext_vector_type(2)));
typedef float f32x2 __attribute__((ext_vector_type(2)));
typedef float f32x16 __attribute__((ext_vector_type(16)));

__device__ __forceinline__ f32x16 mfma32(bf16x8 a, bf16x8 b, f32x16 c) {
  return __builtin_amdgcn_mfma_f32_32x32x16_bf16(a, b, c, 0, 0, 0);
}

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

// Exchange slots start with the odd round tag in the high (S) half of every
// 64-bit word, so no slot reads as a round-0 word before it is written.
__global__ void coop_zero_kernel(unsigned* p, int n, unsigned* status) {
  const int i = blockIdx.x * blockDim.x + threadIdx.x;
  if (i < n) p[i] = (i & 1) ? kTagOdd : 0u;
  if (i == n) *status = 0u;
}

}  // namespace

// KG: largest group size the instance handles (G <= KG); the partners' words of
// a block are loaded together into KG registers.
template <int DP, int KG>
__global__ __launch_bounds__(64 * kNW) void sph_bf16_coop_kernel(CoopArgs a) {
  constexpr int XK = DP / 16;                    // 16-deep k-steps over the x columns (E-GEMM)
  constexpr int XT = DP / 32;                    // 32-wide x tiles of ψ (M-GEMM)
  constexpr int XS = 176;                        // staged row stride (bf16)
  static_assert(DP + kAug <= XS, "row does not fit the staging stride");
  constexpr int JP = DP + 16;                    // statistics columns: x | augmented 0..15
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

  const int tid = threadIdx.x;
  const int wave = tid / 64, lane = tid % 64;
  const int lr = lane % 32, hf = lane / 32;     // 32x32 MFMA: row / component of a tile, k half
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

  // Staged rows start at zero: the lead-in blocks multiply r = 0 by buffers no
  // block has filled yet, which must not hold NaN bit patterns.
  for (int i = tid; i < kNB * kBN * XS / 8; i += NTHR) *reinterpret_cast<uint4*>(xs + 8 * i) = make_uint4(0, 0, 0, 0);
  __syncthreads();
  // Constant augmented columns 8..31 of every staged row: [1 0 0 ...].
  for (int i = tid; i < kNB * kBN * 3; i += NTHR) {
    const int row = i / 3, ch = 1 + i % 3;
    const uint4 w = make_uint4(ch == 1 ? pack2((__bf16)1.f, (__bf16)0.f) : 0u, 0u, 0u, 0u);
    *reinterpret_cast<uint4*>(xs + row * XS + DP + 8 * ch) = w;
  }

  bf16x8 wmu[XK], waug;
  float sc[16];            // log2(e)/σ² of the wave's output components (register v)
  // e = 2^(l2 - m_w) of the two blocks in flight, per block parity, in the
  // accumulator layout (register v: component 8(v/4) + 4hf + v%4 of row lr),
  // kept in fp32 registers until its responsibilities are formed two blocks
  // later (measured 6 % faster per C2 pass than a bf16 copy in LDS, which needs
  // the pack, the read back and the unpack).
  float er[2][16];
  f32x16 accx[XT], acca;
  float mw[2];             // wave row maxima of the two blocks in flight (row lr), per block parity
  unsigned seq = 0;        // blocks this group has exchanged before the current item
  bool dead = false;       // wave 0: a wait timed out; no further waits

  const int items = a.B * a.spb;
  for (int item = grp; item < items; item += a.NG) {
    const int b = item / a.spb, sl = item % a.spb;
    const int64_t rbeg = (int64_t)sl * a.rows_per_item;
    const int64_t rend = (rbeg + a.rows_per_item < N) ? rbeg + a.rows_per_item : N;
    const int nblk = (rend > rbeg) ? (int)((rend - rbeg + kBN - 1) / kBN) : 0;

    // ---- resident component operands (A side of the E-GEMM): lane (lr, hf) holds
    // component kbase + lr, k half hf; padding components get C = -1e30. ----
    {
      const int kk = kbase + lr;
      if (kk < K) {
        const size_t bk = (size_t)b * K + kk;
#pragma unroll
        for (int t = 0; t < XK; ++t)
          wmu[t] = ld16<bf16x8>(reinterpret_cast<const __bf16*>(a.w_mu) + bk * DP + 16 * t + 8 * hf);
        waug = ld16<bf16x8>(reinterpret_cast<const __bf16*>(a.w_aug) + bk * kAug + 8 * hf);
      } else {
#pragma unroll
        for (int e = 0; e < 8; ++e) {
#pragma unroll
          for (int t = 0; t < XK; ++t) wmu[t][e] = (__bf16)0.f;
          waug[e] = (__bf16)((8 * hf + e) == 6 ? -kHuge : 0.f);
        }
      }
#pragma unroll
      for (int v = 0; v < 16; ++v) {
        const int kv = kbase + 8 * (v / 4) + 4 * hf + (v % 4);
        sc[v] = kv < K ? a.w_scale[(size_t)b * K + kv] : 0.f;
      }
#pragma unroll
      for (int xt = 0; xt < XT; ++xt) accx[xt] = f32x16{};
      acca = f32x16{};
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

    // Responsibilities of block i-2 (parity pb, first row rf): r = e · 2^(m_w - lse2),
    // rounded to bf16 and staged row-major for the transposing reads of the M-GEMM.
    // Lane (lr, hf) holds components 8u + 4hf + (0..3), u = 0..3, of row lr.
    auto prep_r = [&](auto PB_, int rf, int nr) {
      constexpr int pb = decltype(PB_)::value;
      const float l2 = lse_s[pb * kBN + lr];     // read unconditionally: no branch around the LDS load
      // rows outside the item (the pipeline's lead-in and drain blocks) get r = 0
      const bool valid = rf + lr >= 0 && rf + lr < nr;
      const float f = valid ? fast_exp2(mw[pb] - l2) : 0.f;
      __bf16* rrow = rs + wave * kBN * kRS + lr * kRS;
#pragma unroll
      for (int u = 0; u < 4; ++u) {
        const float* e4 = er[pb] + 4 * u;
        const uint2 pk = make_uint2(cvt2(e4[0] * f, e4[1] * f), cvt2(e4[2] * f, e4[3] * f));
        *reinterpret_cast<uint2*>(rrow + rswz(lr, 8 * u + 4 * hf)) = pk;
      }
    };
    // Transposing-read addresses of the 32x32x16 operands: lane i of 16-lane group
    // G reads rows 8 (G / 2) + i / 4 (+4) of a k-step and columns 16 (G % 2) + 4 (i % 4).
    const int G16 = lane / 16, i16 = lane % 16;
    const int trow = 8 * (G16 >> 1) + (i16 >> 2), tcol = 16 * (G16 & 1) + 4 * (i16 & 3);
    // M-GEMM of a staged block in two k-steps of 16 rows: acc += rᵀ·ψ, ψ = the staged
    // rows [x | augmented columns 0..31]; hook(k) runs after the k-th MFMA.
    auto mgemm = [&](int bx, auto&& hook) {
      const __bf16* rw = rs + wave * kBN * kRS;
      const __bf16* xw = xs + bx * kBN * XS;
#pragma unroll
      for (int s2 = 0; s2 < 2; ++s2) {
        const int r0 = 16 * s2 + trow;
        const bf16x8 ar = cat(tr16(rw + r0 * kRS + rswz(r0, tcol)), tr16(rw + (r0 + 4) * kRS + rswz(r0 + 4, tcol)));
        bf16x8 bn = cat(tr16(xw + r0 * XS + tcol), tr16(xw + (r0 + 4) * XS + tcol));
#pragma unroll
        for (int xt = 0; xt <= XT; ++xt) {
          const bf16x8 bq = bn;
          if (xt + 1 <= XT) bn = cat(tr16(xw + r0 * XS + 32 * (xt + 1) + tcol), tr16(xw + (r0 + 4) * XS + 32 * (xt + 1) + tcol));
          if (xt < XT) accx[xt] = mfma32(ar, bq, accx[xt]);
          else acca = mfma32(ar, bq, acca);
          hook(s2 * (XT + 1) + xt);
        }
      }
    };
    // E-GEMM of a staged block: lane (lr, hf), register v holds component
    // 8(v/4) + 4hf + v%4 of row lr.  l2 = (log2(e)/σ²)·(x·μ) + [A·‖x‖² + C]: the
    // product of the exact bf16 x and means accumulates in fp32, its factor is
    // applied after the MFMA, and the augmented chunk carries the rest.
    auto egemm = [&](int bx) -> f32x16 {
      const __bf16* xr = xs + bx * kBN * XS + lr * XS + 8 * hf;
      // Operand j of the XK + 1 MFMAs (0: augmented chunk, 1 + t: k-step t) in a
      // rotating three-register-set pipeline, read two MFMAs ahead, so the chain
      // waits for one LDS latency instead of one per MFMA.
      auto opnd = [&](int j) { return ld16<bf16x8>(j == 0 ? xr + DP : xr + 16 * (j - 1)); };
      bf16x8 ob[3];
      ob[0] = opnd(0);
      ob[1] = opnd(1);
      ob[2] = opnd(2);
      __builtin_amdgcn_sched_group_barrier(0x100, 3, 0);
      f32x16 A = f32x16{}, T = f32x16{};
#pragma unroll
      for (int j = 0; j <= XK; ++j) {
        if (j == 0) A = mfma32(waug, ob[0], f32x16{});
        else T = mfma32(wmu[j - 1], ob[j % 3], T);
        if (j + 3 <= XK) ob[j % 3] = opnd(j + 3);
        __builtin_amdgcn_sched_group_barrier(0x008, 1, 0);
        if (j + 3 <= XK) __builtin_amdgcn_sched_group_barrier(0x100, 1, 0);
      }
#pragma unroll
      for (int v = 0; v < 16; ++v) T[v] = fmaf(sc[v], T[v], A[v]);
      return T;
    };
    // E epilogue: wave row maxima m_w, e = 2^(l2 - m_w) (kept in er of the block
    // parity) and the wave's row sums for the workgroup combine; a row's 32
    // components sit in lanes lr and lr + 32.  The exponentials go between the
    // M-GEMM's MFMAs (see step).
    auto row_max = [&](const f32x16& T) {
      float m = T[0];
#pragma unroll
      for (int v = 1; v < 16; ++v) m = fmaxf(m, T[v]);
      return lanes_op<32, true>(m);
    };
    auto lse_sums = [&](float m, auto PB_) {
      constexpr int pb = decltype(PB_)::value;
      const float* e = er[pb];
      float ps[4];
#pragma unroll
      for (int u = 0; u < 4; ++u) ps[u] = (e[4 * u] + e[4 * u + 1]) + (e[4 * u + 2] + e[4 * u + 3]);
      const float sum = lanes_op<32, false>((ps[0] + ps[1]) + (ps[2] + ps[3]));
      mw[pb] = m;
      // Both lanes of a row hold the same values: both store (no branch).
      red_m[(pb * kNW + wave) * RR + lr] = m;
      red_s[(pb * kNW + wave) * RR + lr] = sum;
    };
    if (nblk > 0) { fetch(0); stash(0); }
    if (nblk > 1) { fetch(kBN); stash(1); }
    if (nblk > 2) fetch(2 * kBN);
    __syncthreads();

    // Iteration i of the block pipeline, i = 0 .. nblk + 1 (rounded up to even):
    // the E-GEMM of block i and the M-GEMM of block i-2.  Every iteration runs
    // the same code: the lead-in blocks -2, -1 and the drain blocks nblk,
    // nblk + 1 compute on zeroed or stale staged rows (in bounds) and add
    // nothing, since their rows get r = 0 and take part in no exchange and no
    // log-likelihood.  PB = i & 1, the LDS/register slot parity of blocks i
    // and i-2.
#pragma unroll
    for (int pb = 0; pb < 2; ++pb) {
#pragma unroll
      for (int v = 0; v < 16; ++v) er[pb][v] = 0.f;
      mw[pb] = 0.f;
    }
    auto step = [&](auto PB_, int i) {
      constexpr int PB = decltype(PB_)::value;
      const int r0 = i * kBN;                     // first row of block i in the item
      const bool ahead = i + 2 < nblk;            // block i+2 is in the prefetch registers
      const bool xchg = wave == 0 && i >= 1 && i <= nblk;   // wave 0 collects block i-1
      const bool pubw = wave == 1 && i >= 1 && i <= nblk;   // wave 1 publishes block i-1

      // ---- wave 1: this workgroup's partials of block i-1, published to the group ----
      // (ownM/ownS only seed wave 0's merge below, which overwrites them; written
      // this way the compiled loop measured 2 % faster than without them.)
      float ownM = 0.f, ownS = 0.f;
      if (pubw) {
        if (lane < kBN) {
          constexpr int qb = PB ^ 1;              // parity of block i-1
          // all sixteen partials read before any is used: one LDS latency
          float pm[kNW], ps[kNW];
#pragma unroll
          for (int w = 0; w < kNW; ++w) {
            pm[w] = red_m[(qb * kNW + w) * RR + lane];
            ps[w] = red_s[(qb * kNW + w) * RR + lane];
          }
          float M = pm[0];
#pragma unroll
          for (int w = 1; w < kNW; ++w) M = fmaxf(M, pm[w]);
          float S = 0.f;
#pragma unroll
          for (int w = 0; w < kNW; ++w) S += ps[w] * fast_exp2(pm[w] - M);
          ownM = M;
          ownS = S;
          if (G > 1) {
            const unsigned j = seq + i - 1;
            const uint32_t tagged = (__float_as_uint(S) & ~kTagOdd) | (((j / kRing) & 1) ? kTagOdd : 0u);
            const uint64_t word = (uint64_t)__float_as_uint(M) | ((uint64_t)tagged << 32);
            __hip_atomic_store(gxch + ((j % kRing) * G + mem) * kBN + lane, word, __ATOMIC_RELAXED,
                               __HIP_MEMORY_SCOPE_AGENT);
          }
        }
      }

      // ---- responsibilities of block i-2 with the E-GEMM of block i ----
      f32x16 T;
      prep_r(PB_, r0 - 2 * kBN, nrows);
      T = egemm(i % kNB);

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
      // The staging writes of prep_r and the transposing reads below are LDS
      // operations of this wave only, executed in order; keep the compiler
      // from reordering them.
      __builtin_amdgcn_fence(__ATOMIC_RELEASE, "wavefront");
      __builtin_amdgcn_fence(__ATOMIC_ACQUIRE, "wavefront");
      {
        // The exponentials of block i go between the M-GEMM MFMAs of block i-2:
        // the transcendental unit then works while the matrix core does
        // (measured 2 % faster per C2 pass than after the M-GEMM).
        const float m = row_max(T);
        mgemm((i + kNB - 2) % kNB, [&](int k) {
          if (k < 8) {
            er[PB][2 * k] = fast_exp2(T[2 * k] - m);
            er[PB][2 * k + 1] = fast_exp2(T[2 * k + 1] - m);
          }
        });
        lse_sums(m, PB_);
      }
      __builtin_amdgcn_fence(__ATOMIC_RELEASE, "wavefront");
      __builtin_amdgcn_fence(__ATOMIC_ACQUIRE, "wavefront");

      // ---- wave 0: the group's log-normalisers of block i-1 ----
      if (xchg) {
        float M = ownM, S = ownS;
        if (KG > 1 && G > 1) {
          const bool odd = (jx / kRing) & 1;
          // A word is ready when its tag bit matches the round.
          const uint32_t want = odd ? kTagOdd : 0u;
          auto ready = [&]() {
            uint32_t bad = 0u;
#pragma unroll
            for (int p = 0; p < KG; ++p) {
              const uint32_t hi = (uint32_t)(words[p] >> 32);
              bad |= (p < G) ? ((hi ^ want) & kTagOdd) : 0u;
            }
            return lane >= kBN || bad == 0u;
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
      // The next block's rows are fetched now, a whole iteration before they are
      // staged: waits on the exchange's memory operations during that iteration
      // (the vector memory counter is in order) find them arrived.
      if (i + 3 < nblk) fetch(r0 + 3 * kBN);
      __syncthreads();
    };
    using P0 = std::integral_constant<int, 0>;
    using P1 = std::integral_constant<int, 1>;
    for (int i = 0; i < nblk + 2; i += 2) {
      step(P0{}, i);
      step(P1{}, i + 1);
    }
    seq += (unsigned)nblk;

    // ---- the item's partial statistics (lane (lr, hf), register v: component
    // 8(v/4) + 4hf + v%4 of the wave, feature 32xt + lr) and log-likelihood ----
#pragma unroll
    for (int v = 0; v < 16; ++v) {
      const int kk = kbase + 8 * (v / 4) + 4 * hf + (v % 4);
      if (kk < K) {
        float* dst = a.part_stats + (((size_t)sl * a.B + b) * K + kk) * JP;
#pragma unroll
        for (int xt = 0; xt < XT; ++xt) dst[32 * xt + lr] = accx[xt][v];
        if (lr < 16) dst[DP + lr] = acca[v];
      }
    }
    if (mem == 0 && wave == 0) {
      for (int off = 32; off >= 1; off /= 2) ll += __shfl_xor(ll, off);
      if (lane == 0) a.ll_part[(size_t)b * a.spb + sl] = ll * (double)kLn2;
    }
  }
}

int coop_capacity() {
  // Resident workgroups of the kernel on the current device (cached per device;
  // concurrent first calls store the same value); 256 when no device is visible
  // (workspace sizing on a machine without a GPU).
  static std::atomic<int> cache[64] = {};
  int ndev = 0, dev = 0;
  if (hipGetDeviceCount(&ndev) != hipSuccess || ndev <= 0 || hipGetDevice(&dev) != hipSuccess || dev >= 64) {
    (void)hipGetLastError();
    return 256;
  }
  const int cached = cache[dev].load(std::memory_order_relaxed);
  if (cached > 0) return cached;
  int cus = 0, per = 0;
  if (hipDeviceGetAttribute(&cus, hipDeviceAttributeMultiprocessorCount, dev) != hipSuccess ||
      hipOccupancyMaxActiveBlocksPerMultiprocessor(&per, sph_bf16_coop_kernel<128, 4>, 64 * kNW, 0) != hipSuccess ||
      cus <= 0 || per <= 0) {
    (void)hipGetLastError();
    return 256;
  }
  cache[dev].store(cus * per, std::memory_order_relaxed);
  return cus * per;
}

int launch_sph_bf16_coop(int dp, const CoopArgs& a, hipStream_t s) {
  if (dp != 128 || a.G < 2 || a.G > kMaxCoopGroup) return -1;
  const int grid = a.NG * a.G;
  // The exchange slots (64-bit words) start with the odd round tag, the status word at zero.
  const int nwords = a.NG * kRing * a.G * kBN * 2;
  coop_zero_kernel<<<(nwords + 1 + 255) / 256, 256, 0, s>>>(reinterpret_cast<unsigned*>(a.xch), nwords, a.status);
  const void* fn = a.G <= 2 ? reinterpret_cast<const void*>(sph_bf16_coop_kernel<128, 2>)
                            : reinterpret_cast<const void*>(sph_bf16_coop_kernel<128, 4>);
  // A plain launch of at most the resident capacity: on an otherwise idle device
  // every workgroup is dispatched at once.  Nothing else guarantees it, so the
  // bounded waits are the guard: a member that never meets its partners gives
  // up, sets the status word and drains.
  if (grid > coop_capacity()) return -1;
  CoopArgs args = a;
  void* params[] = {&args};
  const hipError_t e = hipLaunchKernel(fn, dim3(grid), dim3(64 * kNW), params, 0, s);
  if (e != hipSuccess) {
    (void)hipGetLastError();
    return -2;
  }
  return 0;
}

}  // namespace gx
