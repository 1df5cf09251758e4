// Full-covariance inference at D <= 16 and K <= 32 (predict_proba,
// score_samples, labels) by whitening on the bf16 MFMA with split operands.
//
// The tile kernel's E-step forms the row's 136 products x_d x_e and splits each
// into three bf16 parts: at D = 16 that VALU work, not the matrix core, bounds
// it.  Here the quadratic form is a squared norm, (x - μ)ᵀ Σ⁻¹ (x - μ) =
// ‖L⁻¹x - L⁻¹μ‖² (Σ = L Lᵀ; torch_fallback.py:400-432 computes the same value
// expanded, clamped at zero), and only x's 16 values are split.  y = L⁻¹x is a
// 16 x 16 output tile (dims x rows) of v_mfma_f32_16x16x32_bf16 with the six
// products of the split operands (L_h x_h, L_h x_m, L_m x_h, L_h x_l, L_m x_m,
// L_l x_h: the terms of an fp32 product down to 2^-24) laid along k, two per
// MFMA: three MFMAs per 16 rows and component, the accumulator starting at -L⁻¹μ.
//
// One wave takes 4 blocks of 16 rows.  Lane l holds dims 4 (l / 16) + v of row
// l % 16; the four lane groups hold the four quarters of a row's squared norm.
// Components are visited four at a time, component c·KQ + j for lane group c in
// round j (KQ = ceil(K / 4)), and a reduce-scatter over the lane groups (two
// lane swaps) leaves each group the whole norm of its own component: at the end
// lane group c holds the log2 logits of components c·KQ … c·KQ + KQ - 1 of its
// row, so the log-normaliser, the responsibilities (written as contiguous runs)
// and the first argmax need no second pass.  The components' operands (three
// bf16 parts of L⁻¹ in the lane order of the MFMA's A operand, -L⁻¹μ, the log2
// constant) sit in LDS for the whole launch.

#include <math.h>

#include <algorithm>
#include <atomic>

#include "common.hpp"
#include "engine.hpp"

namespace gx {

namespace {

typedef float f32x2 __attribute__((ext_vector_type(2)));
typedef __bf16 bf16x2 __attribute__((ext_vector_type(2)));

constexpr int kWaves = 8;
constexpr int kRB = 4;                     // 16-row blocks per wave
constexpr int kOpElems = 64 * 8;           // one MFMA's A operand: 64 lanes x 8 bf16 (1 KB)

__device__ __forceinline__ f32x4 mfma16(bf16x8 a, bf16x8 b, f32x4 c) {
  return __builtin_amdgcn_mfma_f32_16x16x32_bf16(a, b, c, 0, 0, 0);
}

// The two words of v_permlane{16,32}_swap(x, y): VDST' and SRC0'.  Across the
// swap, lanes of the lower 16- (32-) lane group receive the partner's x in t1,
// lanes of the upper group the partner's y in t0.
__device__ __forceinline__ void swap16(float x, float y, float& t0, float& t1) {
  const auto t = __builtin_amdgcn_permlane16_swap(__float_as_uint(x), __float_as_uint(y), false, false);
  t0 = __uint_as_float(t[0]);
  t1 = __uint_as_float(t[1]);
}
__device__ __forceinline__ void swap32(float x, float y, float& t0, float& t1) {
  const auto t = __builtin_amdgcn_permlane32_swap(__float_as_uint(x), __float_as_uint(y), false, false);
  t0 = __uint_as_float(t[0]);
  t1 = __uint_as_float(t[1]);
}
// Over the four lane groups (lanes l % 16 equal): the same bits in every lane.
__device__ __forceinline__ float sum4(float v) {
  float a, b;
  swap16(v, v, a, b);
  v = a + b;
  swap32(v, v, a, b);
  return a + b;
}
__device__ __forceinline__ float max4(float v) {
  float a, b;
  swap16(v, v, a, b);
  v = fmaxf(a, b);
  swap32(v, v, a, b);
  return fmaxf(a, b);
}

// v = h + m + l exactly, eight values to three bf16x8.
__device__ __forceinline__ void split8(const float (&v)[8], bf16x8& h, bf16x8& m, bf16x8& l) {
#pragma unroll
  for (int p = 0; p < 8; p += 2) {
    const f32x2 a = f32x2{v[p], v[p + 1]};
    const bf16x2 hh = __builtin_convertvector(a, bf16x2);
    const f32x2 r = a - __builtin_convertvector(hh, f32x2);
    const bf16x2 mm = __builtin_convertvector(r, bf16x2);
    const bf16x2 ll = __builtin_convertvector(r - __builtin_convertvector(mm, f32x2), bf16x2);
    h[p] = hh[0];
    h[p + 1] = hh[1];
    m[p] = mm[0];
    m[p + 1] = mm[1];
    l[p] = ll[0];
    l[p + 1] = ll[1];
  }
}

}  // namespace

// ---------------------------------------------------------------------------
// Operands per component: the A operands of the three MFMAs (L⁻¹ zero-padded to
// 16 x 16 and split into bf16 parts h + m + l; MFMA p, lane l = 16 g + r holds
// part PA[p][g / 2] of row r, columns 8 (g % 2) … +7, PA = (h, h | m, h | m, l)),
// -L⁻¹μ and the log2 constant log2 w - ½ log2(e) (D log 2π + log det Σ).
// ---------------------------------------------------------------------------

__global__ __launch_bounds__(64) void full16_pack_kernel(Full16Args a) {
  const int k = blockIdx.x, b = blockIdx.y, t = threadIdx.x;
  const int K = a.K, D = a.D;
  const size_t bk = (size_t)b * K + k;
  const float* X = a.linv + bk * D * D;
  const float* mu = a.means + bk * D;
  __bf16* op = reinterpret_cast<__bf16*>(a.lparts) + bk * 3 * kOpElems;
  for (int e = t; e < 3 * kOpElems; e += 64) {
    const int p = e / kOpElems, l = (e / 8) % 64, u = e % 8;
    const int g = l / 16, i = l % 16, d = 8 * (g & 1) + u;
    const int part = (p == 0) ? 0 : (p == 1 ? ((g >> 1) ? 0 : 1) : ((g >> 1) ? 2 : 1));
    const float v = (i < D && d < D) ? X[i * D + d] : 0.f;
    const __bf16 h = (__bf16)v;
    const float r = v - (float)h;
    const __bf16 m = (__bf16)r;
    op[e] = part == 0 ? h : (part == 1 ? m : (__bf16)(r - (float)m));
  }
  if (t < 16) {
    double acc = 0.0;
    if (t < D)
      for (int j = 0; j <= t; ++j) acc = fma((double)X[t * D + j], (double)mu[j], acc);
    a.bneg[bk * 16 + t] = (float)(-acc);
  }
  if (t == 0) {
    constexpr double kLog2eD = 1.4426950408889634;
    const double c2 = (log((double)a.weights[bk]) - 0.5 * ((double)D * kLog2Pi + (double)a.logdet[bk])) * kLog2eD;
    a.c2[bk] = (float)c2;
  }
}

// ---------------------------------------------------------------------------
// Scores, labels, responsibilities
// ---------------------------------------------------------------------------

// KQ = ceil(K / 4): the components per lane group (a template parameter, so every
// guard on it below is resolved at compile time).
template <int KQ>
__global__ __launch_bounds__(64 * kWaves) void full16_infer_kernel(Full16Args a) {
  __shared__ __align__(16) __bf16 parts[32 * 3 * kOpElems];
  __shared__ __align__(16) float bneg[32 * 16];
  __shared__ float c2s[32];
  const int b = blockIdx.y;
  const int K = a.K, D = a.D;
  const int64_t N = a.N;
  // Stage every component's operands (K <= 32).
  {
    const uint4* src = reinterpret_cast<const uint4*>(reinterpret_cast<const __bf16*>(a.lparts) + (size_t)b * K * 3 * kOpElems);
    uint4* dst = reinterpret_cast<uint4*>(parts);
    for (int i = threadIdx.x; i < K * 3 * kOpElems / 8; i += 64 * kWaves) dst[i] = src[i];
    for (int i = threadIdx.x; i < K * 16; i += 64 * kWaves) bneg[i] = a.bneg[(size_t)b * K * 16 + i];
    for (int i = threadIdx.x; i < K; i += 64 * kWaves) c2s[i] = a.c2[(size_t)b * K + i];
  }
  __syncthreads();

  const int wave = threadIdx.x / 64, lane = threadIdx.x % 64;
  const int lr = lane & 15, g = lane >> 4;    // row of a 16-row block; lane group
  const int half = g & 1, hi = g >> 1;        // dims 8·half … +7 of the operands; product slot
  // The operands are staged once; the workgroup then walks its share of the
  // problem's 512-row tiles (the grid is the device's resident capacity).
  const int64_t ntiles = (N + 16 * kRB * kWaves - 1) / (16 * kRB * kWaves);
  const float* xb = a.x + (size_t)b * N * D;
  // This lane's x values of a tile (row lr of each 16-row block, dims 8·half … +7).
  // (Loading the next tile's during the current one measured no faster.)
  auto load_x = [&](int64_t tile, float (&v)[kRB][8]) {
    const int64_t base = (tile * kWaves + wave) * (16 * kRB);
#pragma unroll
    for (int rb = 0; rb < kRB; ++rb) {
      const int64_t n = base + 16 * rb + lr;
      if (n < N && a.vec_ok) {
        const f32x4 p = *reinterpret_cast<const f32x4*>(xb + (size_t)n * 16 + 8 * half);
        const f32x4 q = *reinterpret_cast<const f32x4*>(xb + (size_t)n * 16 + 8 * half + 4);
#pragma unroll
        for (int u = 0; u < 4; ++u) {
          v[rb][u] = p[u];
          v[rb][4 + u] = q[u];
        }
      } else {
#pragma unroll
        for (int u = 0; u < 8; ++u)
          v[rb][u] = (n < N && 8 * half + u < D) ? xb[(size_t)n * D + 8 * half + u] : 0.f;
      }
    }
  };
  for (int64_t tile = blockIdx.x; tile < ntiles; tile += gridDim.x) {
  const int64_t base = (tile * kWaves + wave) * (16 * kRB);
  float xv[kRB][8];
  load_x(tile, xv);

  // x parts as the B operand of the three MFMAs: products (h, m | h, l | m, h) of
  // slot hi, i.e. B0 = hi ? m : h, B1 = hi ? l : h, B2 = hi ? h : m.
  bf16x8 B0[kRB], B1[kRB], B2[kRB];
#pragma unroll
  for (int rb = 0; rb < kRB; ++rb) {
    bf16x8 h, m, l;
    split8(xv[rb], h, m, l);
    B0[rb] = hi ? m : h;
    B1[rb] = hi ? l : h;
    B2[rb] = hi ? h : m;
  }
  // Every LDS read below is indexed through z, zero but opaque to the compiler
  // and redefined per tile: the component operands are loop-invariant, and
  // without it their loads are hoisted out of the tile loop into registers
  // (hundreds: the kernel then spills).
  int z = 0;
  asm volatile("" : "+v"(z));
  const char* opl = reinterpret_cast<const char*>(parts) + lane * 16 + z;   // this lane's A operands

  float l2v[kRB][KQ];
#pragma unroll
  for (int j = 0; j < KQ; ++j) {
    float q[4][kRB];
#pragma unroll
    for (int c = 0; c < 4; ++c) {
      const int kk = min(c * KQ + j, K - 1);   // past K: a duplicate, masked below
      const char* ok = opl + kk * 3 * 1024;
      const bf16x8 A0 = *reinterpret_cast<const bf16x8*>(ok);
      const bf16x8 A1 = *reinterpret_cast<const bf16x8*>(ok + 1024);
      const bf16x8 A2 = *reinterpret_cast<const bf16x8*>(ok + 2048);
      const f32x4 b0 = *reinterpret_cast<const f32x4*>(&bneg[kk * 16 + 4 * g + z]);
#pragma unroll
      for (int rb = 0; rb < kRB; ++rb) {
        f32x4 acc = mfma16(A0, B0[rb], b0);
        acc = mfma16(A1, B1[rb], acc);
        acc = mfma16(A2, B2[rb], acc);
        q[c][rb] = fmaf(acc[0], acc[0], fmaf(acc[1], acc[1], fmaf(acc[2], acc[2], acc[3] * acc[3])));
      }
    }
    // Reduce-scatter over the lane groups: group c keeps the whole norm of component c.
    const int own = g * KQ + j;
    const float cst = c2s[min(own, K - 1) + z];
#pragma unroll
    for (int rb = 0; rb < kRB; ++rb) {
      float t0, t1, u0, u1;
      swap32(q[0][rb], q[2][rb], t0, t1);
      const float r0 = hi ? q[2][rb] + t0 : q[0][rb] + t1;
      swap32(q[1][rb], q[3][rb], u0, u1);
      const float r1 = hi ? q[3][rb] + u0 : q[1][rb] + u1;
      swap16(r0, r1, t0, t1);
      const float quad = half ? r1 + t0 : r0 + t1;
      l2v[rb][j] = own < K ? fmaf(-0.5f * kLog2e, quad, cst) : -INFINITY;
    }
  }

#pragma unroll
  for (int rb = 0; rb < kRB; ++rb) {
    const int64_t n = base + 16 * rb + lr;
    float m = -INFINITY;
#pragma unroll
    for (int j = 0; j < KQ; ++j) m = fmaxf(m, l2v[rb][j]);
    m = max4(m);
    float e[KQ], s = 0.f;
#pragma unroll
    for (int j = 0; j < KQ; ++j) {
      e[j] = fast_exp2(l2v[rb][j] - m);
      s += e[j];
    }
    s = sum4(s);
    if (n >= N) continue;   // lanes of one row agree: no lane swap below this point
    const float lse = m + __log2f(s);
    if (a.scores && g == 0) a.scores[(size_t)b * N + n] = lse * kLn2;
    if (a.lse2 && g == 0) a.lse2[(size_t)b * N + n] = lse;
    if (a.proba) {
      const float inv = 1.f / s;
      float* pr = a.proba + ((size_t)b * N + n) * K + g * KQ;
      if (KQ == 8 && K == 32) {
        // the group's eight components are a 32-byte aligned run of the row
        *reinterpret_cast<f32x4*>(pr) = f32x4{e[0] * inv, e[1] * inv, e[2] * inv, e[3] * inv};
        *reinterpret_cast<f32x4*>(pr + 4) = f32x4{e[4] * inv, e[5] * inv, e[6] * inv, e[7] * inv};
      } else {
        // (K < 4·KQ: the last group's run stops at K)
#pragma unroll
        for (int j = 0; j < KQ; ++j)
          if (g * KQ + j < K) pr[j] = e[j] * inv;
      }
    }
  }
  if (a.labels) {
    // First argmax: ascending components within a group (strict >), then the
    // lower component index among equal group maxima.
#pragma unroll
    for (int rb = 0; rb < kRB; ++rb) {
      float bv = -INFINITY;
      int bi = g * KQ;
#pragma unroll
      for (int j = 0; j < KQ; ++j)
        if (l2v[rb][j] > bv) {
          bv = l2v[rb][j];
          bi = g * KQ + j;
        }
      float t0, t1, ov;
      float fi = __int_as_float(bi);
      // partner across 16 lanes
      swap16(bv, bv, t0, t1);
      ov = half ? t0 : t1;
      swap16(fi, fi, t0, t1);
      int oi = __float_as_int(half ? t0 : t1);
      if (ov > bv || (ov == bv && oi < bi)) {
        bv = ov;
        bi = oi;
      }
      fi = __int_as_float(bi);
      swap32(bv, bv, t0, t1);
      ov = hi ? t0 : t1;
      swap32(fi, fi, t0, t1);
      oi = __float_as_int(hi ? t0 : t1);
      if (ov > bv || (ov == bv && oi < bi)) {
        bv = ov;
        bi = oi;
      }
      const int64_t n = base + 16 * rb + lr;
      if (n < N && g == 0) a.labels[(size_t)b * N + n] = bi;
    }
  }
  }   // row tiles
}

void launch_full16_pack(const Full16Args& a, hipStream_t s) {
  full16_pack_kernel<<<dim3(a.K, a.B), 64, 0, s>>>(a);
}

// Resident workgroups of the inference kernel on the current device (cached per
// device; concurrent first calls store the same value).
static int full16_capacity() {
  static std::atomic<int> cache[64] = {};
  int dev = 0;
  if (hipGetDevice(&dev) != hipSuccess || dev < 0 || dev >= 64) {
    (void)hipGetLastError();
    return 256;
  }
  const int cached = cache[dev].load(std::memory_order_relaxed);
  if (cached > 0) return cached;
  int cus = 0, per = 0;
  if (hipDeviceGetAttribute(&cus, hipDeviceAttributeMultiprocessorCount, dev) != hipSuccess ||
      hipOccupancyMaxActiveBlocksPerMultiprocessor(&per, reinterpret_cast<const void*>(full16_infer_kernel<8>),
                                                   64 * kWaves, 0) != hipSuccess ||
      cus <= 0 || per <= 0) {
    (void)hipGetLastError();
    return 256;
  }
  cache[dev].store(cus * per, std::memory_order_relaxed);
  return cus * per;
}

void launch_full16_infer(const Full16Args& a, hipStream_t s) {
  const int64_t rows = 16 * kRB * kWaves;
  const int64_t ntiles = (a.N + rows - 1) / rows;
  const int64_t per_problem = std::max<int64_t>(1, (full16_capacity() + a.B - 1) / a.B);
  const unsigned gx = (unsigned)std::min<int64_t>(ntiles, per_problem);
  const dim3 grid(gx, a.B), block(64 * kWaves);
  switch ((a.K + 3) / 4) {
    case 1: full16_infer_kernel<1><<<grid, block, 0, s>>>(a); break;
    case 2: full16_infer_kernel<2><<<grid, block, 0, s>>>(a); break;
    case 3: full16_infer_kernel<3><<<grid, block, 0, s>>>(a); break;
    case 4: full16_infer_kernel<4><<<grid, block, 0, s>>>(a); break;
    case 5: full16_infer_kernel<5><<<grid, block, 0, s>>>(a); break;
    case 6: full16_infer_kernel<6><<<grid, block, 0, s>>>(a); break;
    case 7: full16_infer_kernel<7><<<grid, block, 0, s>>>(a); break;
    default: full16_infer_kernel<8><<<grid, block, 0, s>>>(a); break;
  }
}

}  // namespace gx
