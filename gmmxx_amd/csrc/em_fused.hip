// Fused single-pass EM tile for small K (spherical, bf16 x, K <= 64, D <= 64).
//
// Every wave owns all K components and works through its own contiguous run of
// 32-row blocks, independently of the other waves (no workgroup barriers).
// Per block it
//   1. loads the rows straight from HBM into the E-GEMM operand layout
//      (lane (li, g) holds row 16h + li, columns 32ec + 8g .. +7: a wave reads
//      16 whole rows per instruction) and builds ‖x‖² and the augmented chunk
//      in registers;
//   2. runs the E-GEMM C = W·φᵀ (components x rows) with the augmented k-chunk,
//      which yields the log2 logits directly (see em_sph_bf16.hip);
//   3. reduces each row in registers (in-lane over components, two lane swaps
//      over the four lane groups): m = max_k l, e = 2^(l - m), s = Σ e, and
//      r = e / s -- one exponential per (row, component);
//   4. stages r (row-major) and the rows with their augmented columns in a
//      wave-private LDS region and reads both back with the transposing LDS
//      load as the operands of the M-GEMM acc += rᵀ·ψ.
// Each wave writes one partial statistics tile and one partial log-likelihood
// sum; x is read from HBM once per iteration.

#include "common.hpp"
#include "engine.hpp"

namespace gx {

namespace {

constexpr int kAug = 32;
constexpr float kHuge = 1e30f;
constexpr int kWaves = 4;  // waves per workgroup (independent)

template <typename T>
__device__ __forceinline__ T ld16(const void* p) { return *reinterpret_cast<const T*>(p); }

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

typedef short v4s __attribute__((ext_vector_type(4)));
typedef __bf16 bf16x2 __attribute__((ext_vector_type(2)));

// Transposing LDS read: in each 16-lane group, lane L supplies the address of
// an 8-byte chunk; lane i receives word (i % 4) of the chunks of lanes 4j + i/4.
__device__ __forceinline__ v4s tr16(const __bf16* p) {
  return __builtin_amdgcn_ds_read_tr16_b64_v4i16((__attribute__((address_space(3))) v4s*)p);
}

}  // namespace

template <int DP, int CT>
__global__ __launch_bounds__(64 * kWaves) __attribute__((amdgpu_waves_per_eu(DP * CT >= 256 ? 1 : 2)))
void sph_bf16_fused_kernel(TileArgs a) {
  constexpr int ECH = DP / 32;                  // x chunks of 32 columns
  constexpr int KC = 16 * CT;                   // component slots
  constexpr int JT = DP / 16 + 1;               // ψ = [x | augmented columns 0..15]
  constexpr int JP = 16 * JT;
  // LDS strides (bf16): s = stride/2 dwords ≡ 8 or 24 (mod 32) for the transposing reads.
  constexpr int XS = DP <= 32 ? 80 : 112;
  constexpr int RS = KC <= 32 ? 48 : 80;
  static_assert(DP + 16 <= XS && KC <= RS, "staging strides");

  __shared__ __align__(16) __bf16 xs_all[kWaves * 32 * XS];
  __shared__ __align__(16) __bf16 rs_all[kWaves * 32 * RS];

  const int wave = threadIdx.x / 64, lane = threadIdx.x % 64;
  const int g = lane / 16, li = lane % 16;
  const int b = blockIdx.y;
  const int slice = blockIdx.x * kWaves + wave;
  if (slice >= a.nslices) return;
  const int64_t N = a.N;
  const int K = a.K, D = a.D;
  const int64_t rbeg = (int64_t)slice * a.rows_per_slice;
  const int64_t rend = (rbeg + a.rows_per_slice < N) ? rbeg + a.rows_per_slice : N;
  __bf16* xw = xs_all + wave * 32 * XS;
  __bf16* rw = rs_all + wave * 32 * RS;
  // r rows: the 4-element column chunk is XOR-swizzled by (row / 4) % 4 so that
  // the 16 lanes writing one column of 16 rows, and the transposing reads of 4
  // rows x 4 chunks, both touch 16 distinct bank pairs.
  auto rswz = [](int row, int col) { return col ^ (((row >> 2) & 3) << 2); };

  // ---- components: lane (li, g) holds component 16ct + li, k-group g ----
  bf16x8 whi[CT][ECH], wlo[CT][ECH], waug[CT];
#pragma unroll
  for (int ct = 0; ct < CT; ++ct) {
    const int kk = 16 * ct + li;
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
        waug[ct][s] = (__bf16)((8 * g + s) == 6 ? -kHuge : 0.f);   // C = -1e30: r = 0
      }
    }
  }
  f32x4 acc[CT][JT];
#pragma unroll
  for (int ct = 0; ct < CT; ++ct)
#pragma unroll
    for (int jt = 0; jt < JT; ++jt) acc[ct][jt] = f32x4{0.f, 0.f, 0.f, 0.f};

  // Constant augmented columns 8..15 of the staged rows: [1 0 0 0 0 0 0 0].
  for (int r = lane; r < 32; r += 64)
    *reinterpret_cast<uint4*>(xw + r * XS + DP + 8) = make_uint4(pack2((__bf16)1.f, (__bf16)0.f), 0u, 0u, 0u);

  const __bf16* xb = reinterpret_cast<const __bf16*>(a.x) + (size_t)b * N * D;
  // Row 16h + li, columns 32ec + 8g .. +7 of the block at n0 (zero past the slice end).
  auto load = [&](int64_t n0, uint4 (&v)[2][ECH]) {
    const int last = (int)(rend - 1 - n0);
    const __bf16* blk = xb + (size_t)n0 * D;
#pragma unroll
    for (int h = 0; h < 2; ++h) {
      const int r = 16 * h + li;
      const bool valid = r <= last;
#pragma unroll
      for (int ec = 0; ec < ECH; ++ec) {
        const int c = 32 * ec + 8 * g;
        if (a.vec_ok) {
          const uint4 t = *reinterpret_cast<const uint4*>(blk + (valid ? r : last) * D + c);
          v[h][ec] = valid ? t : make_uint4(0, 0, 0, 0);
        } else {
          union { uint4 u; __bf16 e[8]; } t;
#pragma unroll
          for (int j = 0; j < 8; ++j) t.e[j] = (valid && c + j < D) ? blk[r * D + c + j] : (__bf16)0.f;
          v[h][ec] = t.u;
        }
      }
    }
  };

  double ll = 0.0;
  const int nblk = (rend > rbeg) ? (int)((rend - rbeg + 31) / 32) : 0;
  uint4 cur[2][ECH], nxt[2][ECH];
  if (nblk > 0) load(rbeg, cur);
  for (int ib = 0; ib < nblk; ++ib) {
    const int64_t n0 = rbeg + (int64_t)ib * 32;
    if (ib + 1 < nblk) load(n0 + 32, nxt);
    const int last = (int)(rend - 1 - n0);

    // ‖x‖² per row and the augmented operand (lane group 0: q parts and ones,
    // group 1: the third constant column, groups 2-3: zero).
    bf16x8 xa[2];
#pragma unroll
    for (int h = 0; h < 2; ++h) {
      float q = 0.f;
#pragma unroll
      for (int ec = 0; ec < ECH; ++ec) {
        const uint4 u = cur[h][ec];
        const uint32_t w4[4] = {u.x, u.y, u.z, u.w};
#pragma unroll
        for (int j = 0; j < 4; ++j) {
          const bf16x2 p = __builtin_bit_cast(bf16x2, w4[j]);
          q = __builtin_amdgcn_fdot2_f32_bf16(p, p, q, false);
        }
      }
      q = lanes_op<32, false>(lanes_op<16, false>(q));
      __bf16 qh, qm, ql;
      split3(q, qh, qm, ql);
      const uint4 w0 = make_uint4(pack2(qh, qm), pack2(ql, qh), pack2(qm, qh), pack2((__bf16)1.f, (__bf16)1.f));
      const uint4 w = (g == 0) ? w0 : (g == 1 ? make_uint4(pack2((__bf16)1.f, (__bf16)0.f), 0u, 0u, 0u)
                                              : make_uint4(0u, 0u, 0u, 0u));
      xa[h] = __builtin_bit_cast(bf16x8, w);
      // stage the row (x and augmented columns 0..7) for the ψ operand
      __bf16* row = xw + (16 * h + li) * XS;
#pragma unroll
      for (int ec = 0; ec < ECH; ++ec) *reinterpret_cast<uint4*>(row + 32 * ec + 8 * g) = cur[h][ec];
      if (g == 0) *reinterpret_cast<uint4*>(row + DP) = w0;
    }

    // E-GEMM: T[ct][h] = W(16 comps) · φᵀ(16 rows); lane (li, g): components 16ct + 4g + v of row 16h + li.
    f32x4 T[CT][2];
#pragma unroll
    for (int ct = 0; ct < CT; ++ct)
#pragma unroll
      for (int h = 0; h < 2; ++h) T[ct][h] = mfma_bf16(waug[ct], xa[h], f32x4{0.f, 0.f, 0.f, 0.f});
#pragma unroll
    for (int ec = 0; ec < ECH; ++ec)
#pragma unroll
      for (int ct = 0; ct < CT; ++ct)
#pragma unroll
        for (int h = 0; h < 2; ++h) {
          const bf16x8 xv = __builtin_bit_cast(bf16x8, cur[h][ec]);
          T[ct][h] = mfma_bf16(whi[ct][ec], xv, T[ct][h]);
          T[ct][h] = mfma_bf16(wlo[ct][ec], xv, T[ct][h]);
        }

    // Row log-normaliser and responsibilities.
#pragma unroll
    for (int h = 0; h < 2; ++h) {
      float m = T[0][h][0];
#pragma unroll
      for (int ct = 0; ct < CT; ++ct)
#pragma unroll
        for (int v = 0; v < 4; ++v) m = fmaxf(m, T[ct][h][v]);
      m = lanes_op<32, true>(lanes_op<16, true>(m));
      float s = 0.f;
#pragma unroll
      for (int ct = 0; ct < CT; ++ct)
#pragma unroll
        for (int v = 0; v < 4; ++v) {
          T[ct][h][v] = fast_exp2(T[ct][h][v] - m);
          s += T[ct][h][v];
        }
      s = lanes_op<32, false>(lanes_op<16, false>(s));
      const bool valid = 16 * h + li <= last;
      if (g == 0 && valid) ll += (double)(m + __log2f(s));
      const float inv = valid ? __builtin_amdgcn_rcpf(s) : 0.f;
      const int rr = 16 * h + li;
      __bf16* row = rw + rr * RS;
#pragma unroll
      for (int ct = 0; ct < CT; ++ct) {
        const uint2 p = make_uint2(pack2((__bf16)(T[ct][h][0] * inv), (__bf16)(T[ct][h][1] * inv)),
                                   pack2((__bf16)(T[ct][h][2] * inv), (__bf16)(T[ct][h][3] * inv)));
        *reinterpret_cast<uint2*>(row + 16 * ct + rswz(rr, 4 * g)) = p;
      }
    }
    // The staging writes above and the transposing reads below are LDS operations
    // of this wave only, executed in order; keep the compiler from reordering them.
    __builtin_amdgcn_fence(__ATOMIC_RELEASE, "wavefront");
    __builtin_amdgcn_fence(__ATOMIC_ACQUIRE, "wavefront");

    // M-GEMM: k = data row; lane L of group g reads rows 8g + L/4 (+4), 4 columns at 4(L%4).
    const int rrow = 8 * g + (li >> 2), rcol = 4 * (li & 3);
    bf16x8 ar[CT];
#pragma unroll
    for (int ct = 0; ct < CT; ++ct) {
      const v4s lo = tr16(rw + rrow * RS + 16 * ct + rswz(rrow, rcol));
      const v4s hi = tr16(rw + (rrow + 4) * RS + 16 * ct + rswz(rrow + 4, rcol));
      ar[ct] = __builtin_bit_cast(bf16x8, __builtin_shufflevector(lo, hi, 0, 1, 2, 3, 4, 5, 6, 7));
    }
#pragma unroll
    for (int jt = 0; jt < JT; ++jt) {
      const v4s plo = tr16(xw + rrow * XS + 16 * jt + rcol);
      const v4s phi = tr16(xw + (rrow + 4) * XS + 16 * jt + rcol);
      const bf16x8 bq = __builtin_bit_cast(bf16x8, __builtin_shufflevector(plo, phi, 0, 1, 2, 3, 4, 5, 6, 7));
#pragma unroll
      for (int ct = 0; ct < CT; ++ct) acc[ct][jt] = mfma_bf16(ar[ct], bq, acc[ct][jt]);
    }
    __builtin_amdgcn_fence(__ATOMIC_RELEASE, "wavefront");
    __builtin_amdgcn_fence(__ATOMIC_ACQUIRE, "wavefront");
#pragma unroll
    for (int h = 0; h < 2; ++h)
#pragma unroll
      for (int ec = 0; ec < ECH; ++ec) cur[h][ec] = nxt[h][ec];
  }

  // Partial statistics of this wave's rows: component 16ct + 4g + v, feature 16jt + li.
#pragma unroll
  for (int ct = 0; ct < CT; ++ct)
#pragma unroll
    for (int v = 0; v < 4; ++v) {
      const int kk = 16 * ct + 4 * g + v;
      if (kk < K) {
        float* dst = a.part_stats + (((size_t)slice * a.B + b) * K + kk) * JP;
#pragma unroll
        for (int jt = 0; jt < JT; ++jt) dst[16 * jt + li] = acc[ct][jt][v];
      }
    }
  // Partial log-likelihood (natural log) of this wave's rows.
  for (int off = 32; off >= 1; off /= 2) ll += __shfl_xor(ll, off);
  if (lane == 0) a.ll_part[(size_t)b * a.nslices + slice] = ll * (double)kLn2;
}

int launch_sph_bf16_fused(int dp, int k, const TileArgs& a, int slices, hipStream_t s) {
  const dim3 grid((slices + kWaves - 1) / kWaves, a.B), block(64 * kWaves);
  const int ct = (k + 15) / 16;
  if (dp == 32) {
    switch (ct) {
      case 1: sph_bf16_fused_kernel<32, 1><<<grid, block, 0, s>>>(a); return 0;
      case 2: sph_bf16_fused_kernel<32, 2><<<grid, block, 0, s>>>(a); return 0;
      case 3: case 4: sph_bf16_fused_kernel<32, 4><<<grid, block, 0, s>>>(a); return 0;
      default: return -1;
    }
  }
  if (dp == 64) {
    switch (ct) {
      case 1: sph_bf16_fused_kernel<64, 1><<<grid, block, 0, s>>>(a); return 0;
      case 2: sph_bf16_fused_kernel<64, 2><<<grid, block, 0, s>>>(a); return 0;
      case 3: case 4: sph_bf16_fused_kernel<64, 4><<<grid, block, 0, s>>>(a); return 0;
      default: return -1;
    }
  }
  return -1;
}

}  // namespace gx
