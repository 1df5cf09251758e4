// Fused single-pass EM tile for small K (spherical, bf16 x, K <= 64, D <= 64).
//
// Every wave owns all K components and works through its own contiguous run of
// 32-row blocks, independently of the other waves of its workgroup (they share
// only the staged component operands). The contractions use the 32x32x16 bf16
// MFMA, whose accumulator gives lane l the values of column l % 32 for 16 of
// the 32 rows of a tile: with components as rows and data rows as columns, a
// lane holds 16 components of ONE data row per component tile and its partner
// lane l ^ 32 holds the other 16, so each row reduction is in-lane work plus a
// single lane swap. Per block of 32 rows it
//   1. loads each row straight from HBM (lane l: row l % 32, contiguous columns
//      of half l / 32), forms ‖x‖² and the augmented k-chunk in registers;
//   2. runs the E-GEMM P = x·μ - ‖x‖²/2 + C'_k of the exact bf16 rows and means
//      (fp32 accumulation, the last two terms through the augmented chunk), and
//      scales it to the log2 logits l = s_k·P with s_k = log2(e)/σ²_k in fp32;
//   3. takes the row maximum m, and subtracts it with one more rank-1 MFMA
//      (m split into three bf16 parts, so the shift is exact) instead of one
//      VALU subtraction per element; then e = 2^(l - m), s = Σ e, r = e / s;
//   4. stages r (row-major) and the rows ψ = [x | augmented columns] in a
//      wave-private LDS region and reads both back with the transposing LDS
//      load as the operands of the M-GEMM acc += rᵀ·ψ.
// Each wave writes one partial statistics tile and one partial log-likelihood
// sum; x is read from HBM once per iteration.

#include "common.hpp"
#include "engine.hpp"

namespace gx {

namespace {

constexpr float kHuge = 1e30f;
constexpr int kWaves = kFusedWaves;   // waves per workgroup

typedef float f32x16 __attribute__((ext_vector_type(16)));
typedef short v4s __attribute__((ext_vector_type(4)));
typedef __bf16 bf16x2 __attribute__((ext_vector_type(2)));
typedef float f32x2 __attribute__((ext_vector_type(2)));

template <typename T>
__device__ __forceinline__ T ld16(const void* p) { return *reinterpret_cast<const T*>(p); }

__device__ __forceinline__ f32x16 mfma32(bf16x8 a, bf16x8 b, f32x16 c) {
  return __builtin_amdgcn_mfma_f32_32x32x16_bf16(a, b, c, 0, 0, 0);
}

// The value of the partner lane l ^ 32 combined with this lane's.
template <bool MAX>
__device__ __forceinline__ float half_op(float v) {
  const auto t = __builtin_amdgcn_permlane32_swap(__float_as_uint(v), __float_as_uint(v), false, false);
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

}  // namespace

// KT: 32-component tiles (K <= 32 * KT). VEC: x rows are 16-byte aligned and D == DP.
template <int DP, int KT, bool VEC>
__global__ __launch_bounds__(64 * kWaves) __attribute__((amdgpu_waves_per_eu(DP * KT >= 128 ? 2 : 3)))
void sph_bf16_fused_kernel(TileArgs a) {
  constexpr int XK = DP / 16;                   // k-steps over the x columns
  constexpr int XT = DP / 32;                   // 32-column tiles of x in ψ
  constexpr int KC = 32 * KT;                   // component slots
  constexpr int JP = DP + 16;                   // statistics columns
  // LDS strides (bf16); s = stride / 2 dwords ≡ 8 or 24 (mod 32) keeps the
  // 16-byte accesses and the transposing reads free of bank conflicts.
  constexpr int WS = DP + 16;                   // [μ | scaled augmented constants 0..15]
  constexpr int XS = DP <= 32 ? 80 : 112;       // [x | augmented columns 0..31]
  constexpr int RS = KC <= 32 ? 48 : 80;        // r row
  static_assert(DP + 32 <= XS && KC <= RS, "staging strides");

  // One LDS pool: staged operands while the rows stream, then the workgroup's
  // statistics while the waves' partial tiles are combined.
  constexpr int kPool = KC * WS + kWaves * 32 * (XS + RS);
  static_assert(KC * JP * 2 <= kPool, "combine buffer");
  __shared__ __align__(16) __bf16 pool[kPool];
  __shared__ double llw[kWaves];
  __shared__ __align__(16) float scs[KC];       // s_k = log2(e)/σ²_k (1 for the padding slots)
  __bf16* const ws = pool;
  __bf16* const xs_all = pool + KC * WS;
  __bf16* const rs_all = xs_all + kWaves * 32 * XS;

  const int wave = threadIdx.x / 64, lane = threadIdx.x % 64;
  const int lr = lane % 32, hf = lane / 32;     // data row / component of the tile; k half
  const int b = blockIdx.y;

  // Stage the component operands once per workgroup. Slots past K get μ = 0,
  // s = 1 and C' = -1e30 (augmented column 6), so their responsibilities are 0.
  constexpr int WCH = WS / 8;
  for (int i = threadIdx.x; i < KC * WCH; i += 64 * kWaves) {
    const int kk = i / WCH, c = i % WCH;
    uint4 v = make_uint4(0u, 0u, 0u, 0u);
    if (kk < a.K) {
      const size_t bk = (size_t)b * a.K + kk;
      const __bf16* src = c < DP / 8 ? reinterpret_cast<const __bf16*>(a.w_mu) + bk * DP + 8 * c
                                     : reinterpret_cast<const __bf16*>(a.w_augs) + bk * 16 + 8 * (c - DP / 8);
      v = ld16<uint4>(src);
    } else if (c == DP / 8) {
      v.w = pack2((__bf16)(-kHuge), (__bf16)0.f);   // augmented elements 6 and 7
    }
    *reinterpret_cast<uint4*>(ws + kk * WS + 8 * c) = v;
  }
  for (int kk = threadIdx.x; kk < KC; kk += 64 * kWaves)
    scs[kk] = kk < a.K ? a.w_scale[(size_t)b * a.K + kk] : 1.f;
  __syncthreads();

  // Wave-uniform: keeps the row bookkeeping in scalar registers. A wave past the
  // last slice gets an empty row range (it still takes part in the combine).
  const int slice = __builtin_amdgcn_readfirstlane(blockIdx.x * kWaves + wave);
  const int64_t N = a.N;
  const int D = a.D;
  const int64_t rbeg = slice < a.nslices ? (int64_t)slice * a.rows_per_slice : N;
  const int64_t rend = (rbeg + a.rows_per_slice < N) ? rbeg + a.rows_per_slice : N;
  __bf16* xw = xs_all + wave * 32 * XS;
  __bf16* rw = rs_all + wave * 32 * RS;
  // r rows: the 4-element column chunk is XOR-swizzled by (row / 4) % 4, so that
  // lanes writing one chunk of consecutive rows, and the transposing reads of
  // 4 rows x 4 chunks, touch distinct bank pairs.
  auto rswz = [](int row, int col) { return col ^ (((row >> 2) & 3) << 2); };

  // Constant augmented columns of the staged rows: 8..31 are zero.
  for (int i = lane; i < 32 * 3; i += 64)
    *reinterpret_cast<uint4*>(xw + (i / 3) * XS + DP + 8 + 8 * (i % 3)) = make_uint4(0u, 0u, 0u, 0u);

  // E-GEMM operands of this lane: component 32t + lr, k half hf; x k-step s
  // covers columns 8 (hf XK + s) .. +7, so each lane's x columns are contiguous.
  const __bf16* wl = ws + lr * WS;
  // Rank-1 shift operand: ones in k slots 0..2 for every component.
  const bf16x8 ones3 = __builtin_bit_cast(
      bf16x8, hf == 0 ? make_uint4(pack2((__bf16)1.f, (__bf16)1.f), pack2((__bf16)1.f, (__bf16)0.f), 0u, 0u)
                      : make_uint4(0u, 0u, 0u, 0u));

  f32x16 accx[KT][XT], acca[KT];
#pragma unroll
  for (int t = 0; t < KT; ++t) {
    acca[t] = f32x16{};
#pragma unroll
    for (int xt = 0; xt < XT; ++xt) accx[t][xt] = f32x16{};
  }

  const __bf16* xb = reinterpret_cast<const __bf16*>(a.x) + (size_t)b * N * D;
  // Row lr of the block at n0, chunks hf XK + s. Rows past the slice end must be
  // finite (their responsibilities and log-likelihood terms are masked to zero
  // below): whole-chunk rows use buffer loads bounded by the slice, which return
  // 0 there; padded rows re-read the slice's last row. Every call issues the same
  // loads, so the prefetch below needs no branches.
  // (readfirstlane: the descriptor must live in scalar registers. The builtin
  // returns a signed int: each half is zero-extended through uint32_t, or a low
  // word with bit 31 set would sign-extend into the high word.)
  const uint64_t xaddr = reinterpret_cast<uint64_t>(xb + (size_t)rbeg * D);
  const uint32_t xhi = (uint32_t)__builtin_amdgcn_readfirstlane((int)(uint32_t)(xaddr >> 32));
  const uint32_t xlo = (uint32_t)__builtin_amdgcn_readfirstlane((int)(uint32_t)xaddr);
  const uint64_t xbase = ((uint64_t)xhi << 32) | (uint64_t)xlo;
  const __amdgpu_buffer_rsrc_t xres = __builtin_amdgcn_make_buffer_rsrc(
      reinterpret_cast<void*>(xbase), (short)0, __builtin_amdgcn_readfirstlane((int)((rend - rbeg) * D * 2)),
      0x00020000);
  const int voff = (lr * D + 8 * hf * XK) * 2;
  auto load = [&](int64_t n0, uint4 (&v)[XK]) {
    if constexpr (VEC) {
      const int soff = (int)((n0 - rbeg) * D * 2);
#pragma unroll
      for (int s = 0; s < XK; ++s)
        v[s] = __builtin_bit_cast(uint4, __builtin_amdgcn_raw_buffer_load_b128(xres, voff + 16 * s, soff, 0));
    } else {
      const int64_t nb = n0 < rend ? n0 : n0 - 32;
      const __bf16* blk = xb + (size_t)nb * D;
      const int r = min(lr, (int)(rend - 1 - nb));
#pragma unroll
      for (int s = 0; s < XK; ++s) {
        const int c = 8 * (hf * XK + s);
        // Built as whole dwords so that the loop-carried rows stay in 32-bit registers.
        const uint16_t* src = reinterpret_cast<const uint16_t*>(blk) + (size_t)r * D + c;
        uint32_t w4[4];
#pragma unroll
        for (int j = 0; j < 4; ++j) {
          const uint32_t lo = (c + 2 * j < D) ? src[2 * j] : 0u;
          const uint32_t hi = (c + 2 * j + 1 < D) ? src[2 * j + 1] : 0u;
          w4[j] = lo | (hi << 16);
        }
        v[s] = make_uint4(w4[0], w4[1], w4[2], w4[3]);
      }
    }
  };

  double ll = 0.0;
  const int nblk = (rend > rbeg) ? (int)((rend - rbeg + 31) / 32) : 0;

  // Transposing-read addresses for the 32x32 operands: lane i of 16-lane group G
  // reads rows 8 (G / 2) + i / 4 (+4) of a k-step and columns 16 (G % 2) + 4 (i % 4).
  const int G = lane / 16, i16 = lane % 16;
  const int trow = 8 * (G >> 1) + (i16 >> 2), tcol = 16 * (G & 1) + 4 * (i16 & 3);

  // One block: `cur` holds its rows; the next block's rows are loaded into
  // `nxt`. Two blocks per loop trip, so the two register sets alternate without
  // copies and the prefetch stays in flight while the current block is processed.
  auto block = [&](int64_t n0, uint4 (&cur)[XK], uint4 (&nxt)[XK]) {
    load(n0 + 32, nxt);
    const bool valid = n0 + lr < rend;

    // ‖x‖² of row lr and the augmented operand: k 0..7 (half 0) = q_h q_m q_l q_h q_m q_h 1 1,
    // k 8..15 (half 1) = 1 0 ... 0.
    float q = 0.f;
#pragma unroll
    for (int s = 0; s < XK; ++s) {
      const uint32_t w4[4] = {cur[s].x, cur[s].y, cur[s].z, cur[s].w};
#pragma unroll
      for (int j = 0; j < 4; ++j) {
        const bf16x2 p = __builtin_bit_cast(bf16x2, w4[j]);
        q = __builtin_amdgcn_fdot2_f32_bf16(p, p, q, false);
      }
    }
    q = half_op<false>(q);
    __bf16 qh, qm, ql;
    split3(q, qh, qm, ql);
    const uint4 w0 = make_uint4(pack2(qh, qm), pack2(ql, qh), pack2(qm, qh), pack2((__bf16)1.f, (__bf16)1.f));
    const uint4 w1 = make_uint4(pack2((__bf16)1.f, (__bf16)0.f), 0u, 0u, 0u);
    const bf16x8 phia = __builtin_bit_cast(bf16x8, hf == 0 ? w0 : w1);
    // Stage the row for the ψ operand: x, and augmented columns 0..7 = w0.
    __bf16* row = xw + lr * XS;
#pragma unroll
    for (int s = 0; s < XK; ++s) *reinterpret_cast<uint4*>(row + 8 * (hf * XK + s)) = cur[s];
    if (hf == 0) *reinterpret_cast<uint4*>(row + DP) = w0;

    // E-GEMM: lane l, register v of tile t holds component 32t + 8(v/4) + 4hf + v%4 of row lr.
    // The products of the exact bf16 rows and means accumulate in fp32 after the
    // augmented chunk's -‖x‖²/2 + C'; one fp32 multiply per element scales P to l.
    f32x16 T[KT];
#pragma unroll
    for (int t = 0; t < KT; ++t) {
      const __bf16* wt = wl + 32 * t * WS;
      T[t] = mfma32(ld16<bf16x8>(wt + DP + 8 * hf), phia, f32x16{});
#pragma unroll
      for (int s = 0; s < XK; ++s)
        T[t] = mfma32(ld16<bf16x8>(wt + 8 * (hf * XK + s)), __builtin_bit_cast(bf16x8, cur[s]), T[t]);
#pragma unroll
      for (int j = 0; j < 4; ++j) {
        const float4 sc = *reinterpret_cast<const float4*>(scs + 32 * t + 8 * j + 4 * hf);
        T[t][4 * j] *= sc.x;
        T[t][4 * j + 1] *= sc.y;
        T[t][4 * j + 2] *= sc.z;
        T[t][4 * j + 3] *= sc.w;
      }
    }

    // Row maximum, shifted out by the rank-1 MFMA: T += 1 · (-(m_h + m_m + m_l)).
    float m = T[0][0];
#pragma unroll
    for (int t = 0; t < KT; ++t)
#pragma unroll
      for (int v = 0; v < 16; ++v) m = fmaxf(m, T[t][v]);
    m = half_op<true>(m);
    __bf16 mh, mm, ml;
    split3(-m, mh, mm, ml);
    const bf16x8 phim = __builtin_bit_cast(
        bf16x8, hf == 0 ? make_uint4(pack2(mh, mm), pack2(ml, (__bf16)0.f), 0u, 0u) : make_uint4(0u, 0u, 0u, 0u));
#pragma unroll
    for (int t = 0; t < KT; ++t) T[t] = mfma32(ones3, phim, T[t]);

    // e = 2^(l - m), s = Σ e (pairwise), r = e / s.
#pragma unroll
    for (int t = 0; t < KT; ++t)
#pragma unroll
      for (int v = 0; v < 16; ++v) T[t][v] = fast_exp2(T[t][v]);
    float ps[4 * KT];
#pragma unroll
    for (int t = 0; t < KT; ++t)
#pragma unroll
      for (int u = 0; u < 4; ++u)
        ps[4 * t + u] = (T[t][4 * u] + T[t][4 * u + 1]) + (T[t][4 * u + 2] + T[t][4 * u + 3]);
#pragma unroll
    for (int w = 1; w < 4 * KT; w *= 2)
#pragma unroll
      for (int u = 0; u + w < 4 * KT; u += 2 * w) ps[u] += ps[u + w];
    const float s = half_op<false>(ps[0]);
    if (hf == 0 && valid) ll += (double)(m + __log2f(s));
    const float inv = valid ? __builtin_amdgcn_rcpf(s) : 0.f;
    __bf16* rrow = rw + lr * RS;
#pragma unroll
    for (int t = 0; t < KT; ++t)
#pragma unroll
      for (int u = 0; u < 4; ++u) {
        const uint2 p = make_uint2(cvt2(T[t][4 * u] * inv, T[t][4 * u + 1] * inv),
                                   cvt2(T[t][4 * u + 2] * inv, T[t][4 * u + 3] * inv));
        *reinterpret_cast<uint2*>(rrow + rswz(lr, 32 * t + 8 * u + 4 * hf)) = p;
      }
    // The staging writes above and the transposing reads below are LDS operations
    // of this wave only, executed in order; keep the compiler from reordering them.
    __builtin_amdgcn_fence(__ATOMIC_RELEASE, "wavefront");
    __builtin_amdgcn_fence(__ATOMIC_ACQUIRE, "wavefront");

    // M-GEMM over the 32 rows in two k-steps of 16: acc[t][·] += rᵀ(components of t) · ψ.
#pragma unroll
    for (int s2 = 0; s2 < 2; ++s2) {
      const int r0 = 16 * s2 + trow;
      bf16x8 ar[KT];
#pragma unroll
      for (int t = 0; t < KT; ++t)
        ar[t] = cat(tr16(rw + r0 * RS + rswz(r0, 32 * t + tcol)),
                    tr16(rw + (r0 + 4) * RS + rswz(r0 + 4, 32 * t + tcol)));
#pragma unroll
      for (int xt = 0; xt <= XT; ++xt) {
        const bf16x8 bq = cat(tr16(xw + r0 * XS + 32 * xt + tcol), tr16(xw + (r0 + 4) * XS + 32 * xt + tcol));
#pragma unroll
        for (int t = 0; t < KT; ++t) {
          if (xt < XT) accx[t][xt] = mfma32(ar[t], bq, accx[t][xt]);
          else acca[t] = mfma32(ar[t], bq, acca[t]);
        }
      }
    }
    __builtin_amdgcn_fence(__ATOMIC_RELEASE, "wavefront");
    __builtin_amdgcn_fence(__ATOMIC_ACQUIRE, "wavefront");
  };
  uint4 xa_[XK], xb_[XK];
  if (nblk > 0) load(rbeg, xa_);
  for (int ib = 0; ib < nblk; ib += 2) {
    const int64_t n0 = rbeg + (int64_t)ib * 32;
    block(n0, xa_, xb_);
    __builtin_amdgcn_sched_barrier(0);
    if (ib + 1 < nblk) block(n0 + 32, xb_, xa_);
    __builtin_amdgcn_sched_barrier(0);
  }

  // Combine the waves' partial statistics in LDS in a fixed order (0 + w0 + w1 + ...),
  // then write the workgroup's tile. Lane l, register v of tile t holds component
  // 32t + 8(v/4) + 4hf + v%4 and column lr of an x tile / of the augmented block.
  float* const red = reinterpret_cast<float*>(pool);
  __syncthreads();   // every wave is done with the staging buffers
  for (int i = threadIdx.x; i < KC * JP; i += 64 * kWaves) red[i] = 0.f;
  for (int w = 0; w < kWaves; ++w) {
    __syncthreads();
    if (wave == w) {
#pragma unroll
      for (int t = 0; t < KT; ++t)
#pragma unroll
        for (int v = 0; v < 16; ++v) {
          float* dst = red + (32 * t + 8 * (v / 4) + 4 * hf + (v % 4)) * JP;
#pragma unroll
          for (int xt = 0; xt < XT; ++xt) dst[32 * xt + lr] += accx[t][xt][v];
          if (lr < 16) dst[DP + lr] += acca[t][v];
        }
    }
  }
  // Partial log-likelihood (natural log) of the workgroup's rows, same order.
  for (int off = 32; off >= 1; off /= 2) ll += __shfl_xor(ll, off);
  if (lane == 0) llw[wave] = ll;
  __syncthreads();
  float* out = a.part_stats + ((size_t)blockIdx.x * a.B + b) * a.K * JP;
  for (int i = threadIdx.x; i < a.K * JP; i += 64 * kWaves) out[i] = red[i];
  if (threadIdx.x == 0) {
    double sum = 0.0;
    for (int w = 0; w < kWaves; ++w) sum += llw[w];
    a.ll_part[(size_t)b * gridDim.x + blockIdx.x] = sum * (double)kLn2;
  }
}

template <int DP, int KT>
static void launch_fused(const TileArgs& a, dim3 grid, dim3 block, hipStream_t s) {
  if (a.vec_ok) sph_bf16_fused_kernel<DP, KT, true><<<grid, block, 0, s>>>(a);
  else sph_bf16_fused_kernel<DP, KT, false><<<grid, block, 0, s>>>(a);
}

int launch_sph_bf16_fused(int dp, int k, const TileArgs& a, int slices, hipStream_t s) {
  if (k < 1 || k > 64 || (dp != 32 && dp != 64)) return -1;
  const dim3 grid((slices + kWaves - 1) / kWaves, a.B), block(64 * kWaves);
  const bool one = k <= 32;
  if (dp == 32) {
    if (one) launch_fused<32, 1>(a, grid, block, s);
    else launch_fused<32, 2>(a, grid, block, s);
  } else {
    if (one) launch_fused<64, 1>(a, grid, block, s);
    else launch_fused<64, 2>(a, grid, block, s);
  }
  return 0;
}

}  // namespace gx
