// Greedy k-means++ seeding on a row sample (initialisation of the EM fit).
//
// Restates _kmeans_plus_plus_init_means (gmmxx/torch_fallback.py:1390-1451):
// the first centre is a given row; every later centre is the best of T
// candidates drawn with probability proportional to the squared distance to the
// nearest centre so far (D² sampling through the running cumulative sum), "best"
// meaning the smallest potential Σ_i min(closest_i, ‖s_i - c‖²).  The random
// numbers (first row, uniform draws) are inputs, so the result is a pure
// function of them.
//
// Per step two launches: kpp_trial_kernel (many workgroups over the rows:
// candidate distances and per-block partial potentials) and kpp_pick_kernel
// (one workgroup per batch: pick the candidate, update the closest distances,
// then scan them and draw the next step's candidates).  The row sample is read
// once per step (T distances per row from one read); everything else is
// O(S) per step.

#include "common.hpp"
#include "engine.hpp"

namespace gx {

namespace {

constexpr int kTrialThreads = 256;   // rows per trial workgroup
constexpr int kPickThreads = 1024;

__device__ __forceinline__ float wave_sum(float v) {
#pragma unroll
  for (int off = 32; off >= 1; off /= 2) v += __shfl_xor(v, off);
  return v;
}

// Squared Euclidean distances of one row to `t_count` LDS-resident candidates
// (direct differences, as the reference computes them).
template <bool VEC>
__device__ __forceinline__ void row_dists(const float* __restrict__ row, const float* cand, int D, int t_count,
                                          float (&acc)[kKppMaxTrials]) {
#pragma unroll
  for (int t = 0; t < kKppMaxTrials; ++t) acc[t] = 0.f;
  if constexpr (VEC) {
    for (int d = 0; d < D; d += 4) {
      const float4 v = *reinterpret_cast<const float4*>(row + d);
#pragma unroll
      for (int t = 0; t < kKppMaxTrials; ++t) {
        if (t < t_count) {
          const float4 c = *reinterpret_cast<const float4*>(cand + t * D + d);
          const float a = v.x - c.x, b = v.y - c.y, e = v.z - c.z, f = v.w - c.w;
          acc[t] = fmaf(a, a, acc[t]);
          acc[t] = fmaf(b, b, acc[t]);
          acc[t] = fmaf(e, e, acc[t]);
          acc[t] = fmaf(f, f, acc[t]);
        }
      }
    }
  } else {
    for (int d = 0; d < D; ++d) {
      const float v = row[d];
#pragma unroll
      for (int t = 0; t < kKppMaxTrials; ++t) {
        if (t < t_count) {
          const float a = v - cand[t * D + d];
          acc[t] = fmaf(a, a, acc[t]);
        }
      }
    }
  }
}

// closest_i = ‖s_i - s_first‖²; workgroup (0, b) also writes centre 0.
__global__ __launch_bounds__(kTrialThreads) void kpp_first_kernel(KppArgs a) {
  extern __shared__ float cand[];
  const int b = blockIdx.y;
  const float* sample = a.sample + (size_t)b * a.S * a.D;
  const int64_t f = min<int64_t>(max<int64_t>(a.first[b], 0), a.S - 1);
  for (int d = threadIdx.x; d < a.D; d += blockDim.x) {
    const float v = sample[(size_t)f * a.D + d];
    cand[d] = v;
    if (blockIdx.x == 0) a.centers[(size_t)b * a.K * a.D + d] = v;
  }
  __syncthreads();
  const int i = blockIdx.x * kTrialThreads + threadIdx.x;
  if (i < a.S) {
    float acc[kKppMaxTrials];
    if (a.vec) row_dists<true>(sample + (size_t)i * a.D, cand, a.D, 1, acc);
    else row_dists<false>(sample + (size_t)i * a.D, cand, a.D, 1, acc);
    a.closest[(size_t)b * a.S + i] = acc[0];
  }
}

// Distances of every row to the step's T candidates (kept for the pick) and
// the block's partial potentials Σ min(closest, dist) per candidate.
__global__ __launch_bounds__(kTrialThreads) void kpp_trial_kernel(KppArgs a) {
  extern __shared__ float cand[];
  __shared__ float red[kTrialThreads / 64][kKppMaxTrials];
  const int b = blockIdx.y, T = a.T;
  const float* sample = a.sample + (size_t)b * a.S * a.D;
  for (int e = threadIdx.x; e < T * a.D; e += blockDim.x) {
    const int t = e / a.D, d = e % a.D;
    cand[e] = sample[(size_t)a.cand[b * kKppMaxTrials + t] * a.D + d];
  }
  __syncthreads();
  const int i = blockIdx.x * kTrialThreads + threadIdx.x;
  float acc[kKppMaxTrials];
  if (i < a.S) {
    if (a.vec) row_dists<true>(sample + (size_t)i * a.D, cand, a.D, T, acc);
    else row_dists<false>(sample + (size_t)i * a.D, cand, a.D, T, acc);
    const float cl = a.closest[(size_t)b * a.S + i];
#pragma unroll
    for (int t = 0; t < kKppMaxTrials; ++t) {
      if (t < T) {
        a.dist[((size_t)b * kKppMaxTrials + t) * a.S + i] = acc[t];
        acc[t] = fminf(cl, acc[t]);
      }
    }
  } else {
#pragma unroll
    for (int t = 0; t < kKppMaxTrials; ++t) acc[t] = 0.f;
  }
  const int wave = threadIdx.x / 64, lane = threadIdx.x % 64;
#pragma unroll
  for (int t = 0; t < kKppMaxTrials; ++t) {
    if (t < T) {
      const float s = wave_sum(acc[t]);
      if (lane == 0) red[wave][t] = s;
    }
  }
  __syncthreads();
  if (threadIdx.x < T) {
    float s = 0.f;
    for (int w = 0; w < kTrialThreads / 64; ++w) s += red[w][threadIdx.x];
    a.pot_part[((size_t)b * a.nblk + blockIdx.x) * kKppMaxTrials + threadIdx.x] = s;
  }
}

// Step `step` (>= 1): the candidate of least potential (first on ties) becomes
// centre `step` and the closest distances take its column.  Then, when
// step + 1 < K, the next step's candidates: thread j owns rows [jR, jR + R),
// the chunk sums are scanned across the workgroup, and draw u·total lands on
// the first row whose running sum reaches it (searchsorted, left side), the
// last row when it exceeds the total, row 0 when the total is 0.
__global__ __launch_bounds__(kPickThreads) void kpp_pick_kernel(KppArgs a, int step) {
  __shared__ float scan[kPickThreads];
  __shared__ int best_s;
  const int b = blockIdx.x, tid = threadIdx.x, T = a.T;
  const float* sample = a.sample + (size_t)b * a.S * a.D;
  float* closest = a.closest + (size_t)b * a.S;
  int* cand = a.cand + b * kKppMaxTrials;
  const int R = (a.S + kPickThreads - 1) / kPickThreads;
  const int i0 = min(a.S, tid * R), i1 = min(a.S, i0 + R);

  if (step >= 1) {
    if (tid == 0) {
      double best_v = 0.0;
      int best = 0;
      for (int t = 0; t < T; ++t) {
        double p = 0.0;
        for (int k = 0; k < a.nblk; ++k) p += (double)a.pot_part[((size_t)b * a.nblk + k) * kKppMaxTrials + t];
        if (t == 0 || p < best_v) { best_v = p; best = t; }
      }
      best_s = best;
    }
    __syncthreads();
    const int best = best_s;
    const int64_t row = cand[best];
    for (int d = tid; d < a.D; d += kPickThreads)
      a.centers[((size_t)b * a.K + step) * a.D + d] = sample[(size_t)row * a.D + d];
    const float* db = a.dist + ((size_t)b * kKppMaxTrials + best) * a.S;
    for (int i = i0; i < i1; ++i) closest[i] = fminf(closest[i], db[i]);
    __syncthreads();   // every thread has read cand[] before it is rewritten below
  }
  if (step + 1 >= a.K) return;

  float cs = 0.f;
  for (int i = i0; i < i1; ++i) cs += closest[i];
  scan[tid] = cs;
  __syncthreads();
  // inclusive Hillis-Steele scan of the chunk sums
  for (int off = 1; off < kPickThreads; off *= 2) {
    const float v = (tid >= off) ? scan[tid - off] : 0.f;
    __syncthreads();
    scan[tid] += v;
    __syncthreads();
  }
  const float incl = scan[tid];
  const float prev = (tid == 0) ? 0.f : scan[tid - 1];
  const float total = scan[kPickThreads - 1];
  const float* u = a.draws + ((size_t)b * (a.K - 1) + step) * T;
  for (int t = 0; t < T; ++t) {
    if (!(total > 0.f)) {
      if (tid == 0) cand[t] = 0;
      continue;
    }
    const float target = u[t] * total;
    if (!(target <= total)) {   // beyond the total (or NaN): clamp to the last row
      if (tid == 0) cand[t] = a.S - 1;
      continue;
    }
    if (incl >= target && (tid == 0 || prev < target) && i1 > i0) {
      float run = prev;
      int idx = i1 - 1;
      for (int i = i0; i < i1; ++i) {
        run += closest[i];
        if (run >= target) { idx = i; break; }
      }
      cand[t] = idx;
    }
  }
}

}  // namespace

int64_t kpp_workspace_bytes(int B, int S, int K, int T) {
  (void)K;
  (void)T;
  const int64_t nblk = (S + kTrialThreads - 1) / kTrialThreads;
  auto up = [](int64_t v) { return (v + 255) / 256 * 256; };
  return up((int64_t)B * S * 4) + up((int64_t)B * kKppMaxTrials * S * 4) +
         up((int64_t)B * nblk * kKppMaxTrials * 4) + up((int64_t)B * kKppMaxTrials * 4);
}

void kpp_bind_workspace(KppArgs& a, void* ws) {
  a.nblk = (a.S + kTrialThreads - 1) / kTrialThreads;
  auto up = [](int64_t v) { return (v + 255) / 256 * 256; };
  char* p = static_cast<char*>(ws);
  a.closest = reinterpret_cast<float*>(p);
  p += up((int64_t)a.B * a.S * 4);
  a.dist = reinterpret_cast<float*>(p);
  p += up((int64_t)a.B * kKppMaxTrials * a.S * 4);
  a.pot_part = reinterpret_cast<float*>(p);
  p += up((int64_t)a.B * a.nblk * kKppMaxTrials * 4);
  a.cand = reinterpret_cast<int*>(p);
}

void launch_kpp(const KppArgs& a, hipStream_t s) {
  const dim3 rows(a.nblk, a.B);
  kpp_first_kernel<<<rows, kTrialThreads, a.D * sizeof(float), s>>>(a);
  kpp_pick_kernel<<<a.B, kPickThreads, 0, s>>>(a, 0);
  for (int step = 1; step < a.K; ++step) {
    kpp_trial_kernel<<<rows, kTrialThreads, a.T * a.D * sizeof(float), s>>>(a);
    kpp_pick_kernel<<<a.B, kPickThreads, 0, s>>>(a, step);
  }
}

}  // namespace gx
