// C-ABI entry points of libgmmxx_hip.so (declared in include/gmmxx_hip.h).
//
// Each call plans the launch geometry for the problem, carves the caller's
// workspace, and enqueues the kernels of one operation on the caller's stream.
// Nothing is allocated and nothing synchronises.

#include <stdint.h>

#include <stdio.h>
#include <stdlib.h>
#include <string.h>

#include <algorithm>
#include <mutex>
#include <string>

#include "common.hpp"
#include "engine.hpp"
#include "gmmxx_hip.h"
#include "params.hpp"

namespace {

using namespace gx;

thread_local std::string g_last_error;

// Device scratch of the no-allocation entry point (gmmxx_hip_em_step_noalloc):
// the workspace of problems up to kScratchBytes, one copy per device for the
// life of the process.  In host code `scratch` names a host-side stand-in:
// its device address comes from hipGetSymbolAddress, once per device, and
// only that address is handed to kernels.
constexpr int64_t kScratchBytes = int64_t(64) << 20;
constexpr int kMaxDevices = 64;
static __device__ __align__(256) unsigned char scratch[kScratchBytes];
std::mutex g_scratch_mu;
void* g_scratch_ptr[kMaxDevices] = {};

int fail(int code, const std::string& msg) {
  g_last_error = msg;
  return code;
}

struct Plan {
  int cov = 0, bf = 0, B = 0, D = 0, K = 0;
  int64_t N = 0;
  int DP = 0, EP = 0, JP = 0, nk_col = 0, sq_col = 0, sq_n = 0, CW = 0, nw = 0, ktiles = 0, slices = 0, cblocks = 0;
  int lnw = 0, lktiles = 0;  // waves / component tiles of the plain log-normaliser pass (MODE_LSE)
  bool fused = false;        // EM iteration as one fused pass (small K; em_fused.hip)
  bool coop = false;         // EM iteration as one cooperative pass (spherical bf16, D = 128; em_coop.hip)
  bool single = false;       // EM iteration as one tile pass (fp32 x, all K in one workgroup; MODE_STATS_LSE)
  bool xch = false;          // EM iteration as one tile pass whose 2..4 component tiles exchange row partials
  int xslices = 0;           // xch: row slices per batch (grid xslices·ktiles x B, all resident)
  int64_t xrows = 0;         // xch: rows per slice
  int cG = 0, cNG = 0, cspb = 0;   // coop: workgroups per group, groups, row items per batch
  int64_t crows = 0;         // coop: rows per item
  int fslices = 0;           // fused: one wave per row slice
  int fparts = 0;            // fused: partial results (one per workgroup of kFusedWaves slices)
  int64_t frows = 0;
  int64_t rows_per_slice = 0;
  int gram_slices = 0;
  int64_t gram_rows = 0;
  int chol_m = 0;
  size_t o_whi = 0, o_wlo = 0, o_waug = 0, o_wmu = 0, o_wsc = 0, o_waugs = 0, o_cconst = 0, o_covs_used = 0, o_rowq = 0, o_lse2 = 0, o_pms = 0, o_pidx = 0;
  size_t o_xch = 0, o_flags = 0;
  // full covariance at D > 16 (whitening E-step, weighted-Gram statistics)
  bool fw = false;
  int pdt = 0;   // param_dtype
  int fw_eblk = 0, fw_slices = 0;
  int64_t fw_rows = 0;
  size_t o_lpack = 0, o_lpaug = 0, o_l2w = 0, o_linv = 0;
  // full covariance at D <= 16, K <= 32: whitening inference (score, labels, proba)
  bool w16 = false;
  size_t o_w16parts = 0, o_w16b = 0, o_w16c = 0;
  size_t o_rowaux = 0, o_pstats = 0, o_stats = 0, o_ll = 0, o_first = 0, o_lbuf = 0, o_prec = 0, o_logdet = 0,
         o_gram = 0, total = 0;
};

constexpr int kTargetWaves = 2048;      // one round at two resident waves per SIMD (the tile kernels'
                                        // usual occupancy; 4096 measured 4 % slower at C4, 8192 6 %)
constexpr int kMinBlocksPerSlice = 3;  // row blocks of one slice (bounds the partial-statistics count)

int dp_for(int64_t d) {
  const int dps[] = {16, 32, 64, 128};
  for (int v : dps)
    if (d <= v) return v;
  return -1;
}

int plan_problem(const gmmxx_problem* p, Plan* pl) {
  if (!p) return fail(GMMXX_ERR_INVALID_ARGUMENT, "problem descriptor is NULL");
  if (p->covariance_type < 0 || p->covariance_type > 3)
    return fail(GMMXX_ERR_INVALID_ARGUMENT, "covariance_type must be 0..3");
  if (p->x_dtype != GMMXX_F32 && p->x_dtype != GMMXX_BF16)
    return fail(GMMXX_ERR_INVALID_ARGUMENT, "x_dtype must be GMMXX_F32 or GMMXX_BF16");
  if (p->param_dtype != GMMXX_F32 && p->param_dtype != GMMXX_BF16 && p->param_dtype != GMMXX_F16)
    return fail(GMMXX_ERR_INVALID_ARGUMENT, "param_dtype must be GMMXX_F32, GMMXX_BF16 or GMMXX_F16");
  if (p->x_dtype == GMMXX_BF16 && p->param_dtype == GMMXX_F16)
    return fail(GMMXX_ERR_INVALID_ARGUMENT, "bf16 x keeps its means in bf16: param_dtype must not be GMMXX_F16");
  if (p->reserved != 0) return fail(GMMXX_ERR_INVALID_ARGUMENT, "reserved must be 0");
  if (p->B < 1 || p->N < 1 || p->D < 1 || p->K < 1)
    return fail(GMMXX_ERR_INVALID_ARGUMENT, "B, N, D and K must be positive");
  if (p->B > 65535) return fail(GMMXX_ERR_UNSUPPORTED, "B > 65535");
  if (p->K > 65536) return fail(GMMXX_ERR_UNSUPPORTED, "K > 65536");
  if (p->N > (int64_t)1 << 40) return fail(GMMXX_ERR_UNSUPPORTED, "N too large");
  Plan& q = *pl;
  q.cov = p->covariance_type;
  q.bf = p->x_dtype == GMMXX_BF16;
  q.pdt = p->param_dtype;
  q.B = (int)p->B;
  q.N = p->N;
  q.D = (int)p->D;
  q.K = (int)p->K;
  if (q.bf && q.cov != SPH) return fail(GMMXX_ERR_UNSUPPORTED, "bf16 input is supported for spherical only");
  const int dmax = 128;
  if (p->D > dmax) return fail(GMMXX_ERR_UNSUPPORTED, "D exceeds the supported maximum for this covariance type");
  q.DP = dp_for(q.D);
  // Full covariance beyond D = 16: the whitening kernels of em_full_wide.hip
  // (the tile kernel's augmented features are built for D = 16).
  q.fw = q.cov == FULL && q.DP > 16;
  // (the whitening E-step's per-problem workgroup count is an int: 128 rows each)
  if (q.fw && q.N > ((int64_t)1 << 36)) return fail(GMMXX_ERR_UNSUPPORTED, "N too large for full covariance at D > 16");
  // Full covariance at D <= 16 with every component in one wave: inference by
  // whitening (em_full_infer.hip) instead of the tile kernel's 136 products per
  // row.  GMMXX_HIP_NO_WHITEN=1 keeps the tile kernels (the tests compare both).
  const char* no_whiten = getenv("GMMXX_HIP_NO_WHITEN");
  q.w16 = q.cov == FULL && q.DP == 16 && q.K <= kFull16MaxK && !(no_whiten && no_whiten[0] == '1');
  const bool sph_bf = q.bf && q.cov == SPH;          // dedicated kernel, DP >= 32
  if (sph_bf) q.DP = std::max(q.DP, 32);
  const int S = q.DP * (q.DP + 1) / 2;
  const int E = (q.cov == SPH || q.cov == TIED) ? q.DP : (q.cov == DIAG ? 2 * q.DP : S + q.DP);
  const int J = (q.cov == SPH) ? q.DP + 3 : (q.cov == DIAG ? 2 * q.DP + 1 : (q.cov == TIED ? q.DP + 1 : q.DP + S + 1));
  q.EP = q.fw ? 0 : round_up(E, 32);
  q.JP = round_up(J, 16);
  q.nk_col = (q.cov == SPH) ? q.DP : (q.cov == DIAG ? 2 * q.DP : (q.cov == TIED ? q.DP : q.DP + S));
  q.sq_col = q.DP + 1;
  q.sq_n = 2;
  if (sph_bf) {
    // statistics row = [Σr·x | Σr·(augmented columns q_h q_m q_l q_h q_m q_h 1 1 1 0 ...)]
    q.nk_col = q.DP + 6;
    q.sq_col = q.DP;
    q.sq_n = 3;
  }
  q.CW = tile_cw(q.cov, q.DP, q.bf);
  // Waves per workgroup: a power of two (the cross-wave combine reduces lane groups).
  const int need = (q.K + q.CW - 1) / q.CW;
  q.nw = need <= 1 ? 1 : (need <= 2 ? 2 : (need <= 4 ? 4 : 8));
  // bf16 spherical: at least 2 waves; at D = 128 always 8 (the 2- and 4-wave
  // variants prefetch several chunks per thread and run out of registers).
  if (sph_bf) q.nw = q.DP >= 128 ? 8 : std::max(q.nw, 2);
  q.ktiles = (q.K + q.nw * q.CW - 1) / (q.nw * q.CW);
  // The bf16 D = 128 log-normaliser pass runs 16-wave workgroups (512 components)
  // when K needs more than one 8-wave tile: the staged rows are shared by twice
  // the waves and four waves per SIMD hide each other's VALU work.
  q.lnw = (sph_bf && q.DP == 128 && q.K > 8 * q.CW) ? 16 : q.nw;
  q.lktiles = (q.K + q.lnw * q.CW - 1) / (q.lnw * q.CW);
  const int64_t row_blocks = (q.N + kBN - 1) / kBN;
  const int64_t target_blocks = (kTargetWaves + q.nw - 1) / q.nw;
  int64_t slices = std::max<int64_t>(1, (target_blocks + (int64_t)q.ktiles * q.B - 1) / ((int64_t)q.ktiles * q.B));
  slices = std::min(slices, std::max<int64_t>(1, row_blocks / kMinBlocksPerSlice));
  q.rows_per_slice = ((q.N + slices - 1) / slices + kBN - 1) / kBN * kBN;
  q.slices = (int)((q.N + q.rows_per_slice - 1) / q.rows_per_slice);
  q.cblocks = combine_blocks(q.N);
  // Fused single pass: spherical bf16 with every component in one wave's registers.
  q.fused = sph_bf && q.DP <= 64 && q.K <= 64;
  if (q.fused) {
    // ~6144 waves: two full rounds at three resident waves per SIMD.
    int64_t fs = std::max<int64_t>(1, (6144 + q.B - 1) / q.B);
    fs = std::min(fs, std::max<int64_t>(1, row_blocks / kMinBlocksPerSlice));
    // The kernel addresses a slice with 32-bit buffer offsets: keep it under 1 GiB.
    fs = std::max<int64_t>(fs, (q.N * q.D * 2 + (int64_t(1) << 30) - 1) >> 30);
    q.frows = ((q.N + fs - 1) / fs + kBN - 1) / kBN * kBN;
    q.fslices = (int)((q.N + q.frows - 1) / q.frows);
    q.fparts = (q.fslices + kFusedWaves - 1) / kFusedWaves;
  }
  // Cooperative single pass: spherical bf16 at D = 128 with 256 < K <= 1024
  // (groups of 2..4 workgroups; at one group member and at eight the two-pass
  // kernels measured faster).  Group members must be co-resident, so the grid is
  // the device's resident capacity rounded to whole groups (multiples of 8
  // groups keep each group on one XCD).  GMMXX_HIP_NO_COOP=1 selects the
  // two-pass kernels instead.
  const char* no_coop = getenv("GMMXX_HIP_NO_COOP");
  q.coop = sph_bf && q.DP == 128 && q.D == 128 && q.K > kCoopComps && q.K <= kCoopComps * kMaxCoopGroup &&
           !(no_coop && no_coop[0] == '1');
  if (q.coop) {
    q.cG = (q.K + kCoopComps - 1) / kCoopComps;
    int ng = coop_capacity() / q.cG;
    if (ng >= 8) ng -= ng % 8;
    q.cNG = ng;
    q.coop = ng >= 1;
  }
  if (q.coop) {
    int64_t spb = std::max<int64_t>(1, q.cNG / q.B);
    spb = std::min(spb, std::max<int64_t>(1, row_blocks / kMinBlocksPerSlice));
    // An item is addressed with 32-bit offsets: keep it under 2^30 bytes of x.
    spb = std::max<int64_t>(spb, (q.N * q.DP * 2 + (int64_t(1) << 30) - 1) >> 30);
    q.crows = ((q.N + spb - 1) / spb + kBN - 1) / kBN * kBN;
    q.cspb = (int)((q.N + q.crows - 1) / q.crows);
  }
  // One-tile single pass: the workgroup holds every component, so the tile kernel
  // forms the row log-normalisers itself (diag at D = 128 keeps two passes: its
  // statistics kernel is at the register limit).  GMMXX_HIP_NO_SINGLE=1 selects
  // the two passes.
  const char* no_single = getenv("GMMXX_HIP_NO_SINGLE");
  q.single = !sph_bf && !q.fw && q.ktiles == 1 && !(q.cov == DIAG && q.DP >= 128) &&
             !(no_single && no_single[0] == '1');
  // Exchange single pass (fp32 spherical, tied, diag at D <= 64; 2..4 component
  // tiles of 8 waves): the workgroups of a row slice swap per-row (max, sum)
  // partials, so x is read once per iteration.  They must be co-resident: the
  // grid is at most the device's resident capacity of that kernel.
  // GMMXX_HIP_NO_XCH=1 selects the two passes.
  const char* no_xch = getenv("GMMXX_HIP_NO_XCH");
  q.xch = !q.bf && (q.cov == SPH || q.cov == TIED || (q.cov == DIAG && q.DP <= 64)) && q.ktiles >= 2 &&
          q.ktiles <= kMaxCoopGroup && q.nw == 8 && !(no_xch && no_xch[0] == '1');
  if (q.xch) {
    int64_t xs = tile_xch_capacity(q.cov, q.DP) / ((int64_t)q.ktiles * q.B);
    xs = std::min(xs, std::max<int64_t>(1, row_blocks / kMinBlocksPerSlice));
    q.xch = xs >= 1;
    if (q.xch) {
      q.xrows = ((q.N + xs - 1) / xs + kBN - 1) / kBN * kBN;
      q.xslices = (int)((q.N + q.xrows - 1) / q.xrows);
    }
  }
  // XᵀX: about 512 workgroups in all, slices of whole 16-row groups (the kernel's
  // four waves take four rows at a time).
  int64_t gs = std::max<int64_t>(1, std::min<int64_t>((512 + q.B - 1) / q.B, (q.N + 255) / 256));
  q.gram_rows = ((q.N + gs - 1) / gs + 15) / 16 * 16;
  q.gram_slices = (int)((q.N + q.gram_rows - 1) / q.gram_rows);
  q.chol_m = (q.cov == TIED) ? q.B : (q.cov == FULL ? q.B * q.K : 0);
  if (q.fw) {
    // E-step: one wave per 32-row block.  Statistics: workgroups of four waves
    // (four components; at D = 128 two components of two waves) over row slices,
    // as many as one round of resident waves: 8, 4 and 2 waves per SIMD at
    // DP = 32, 64 and 128 (the kernels' register counts), so 2048, 1024 and 512
    // workgroups (at D = 64, 2048 measured 5 % slower per EM iteration).
    q.fw_eblk = fw_eblocks(q.N);
    const int64_t groups = (int64_t)(q.DP == 128 ? (q.K + 1) / 2 : (q.K + 3) / 4) * q.B;
    const int64_t target = q.DP == 32 ? 2048 : (q.DP == 64 ? 1024 : 512);
    int64_t fs = std::max<int64_t>(1, (target + groups - 1) / groups);
    fs = std::min(fs, std::max<int64_t>(1, row_blocks / kMinBlocksPerSlice));
    q.fw_rows = ((q.N + fs - 1) / fs + kBN - 1) / kBN * kBN;
    q.fw_slices = (int)((q.N + q.fw_rows - 1) / q.fw_rows);
  }

  size_t off = 0;
  auto take = [&](size_t bytes) {
    const size_t o = off;
    off += (bytes + 255) / 256 * 256;
    return o;
  };
  const size_t BK = (size_t)q.B * q.K, BN = (size_t)q.B * q.N;
  q.o_whi = take(BK * q.EP * (q.bf ? 2 : 4));
  q.o_wlo = take(q.bf ? BK * q.EP * 2 : 0);
  q.o_waug = take(sph_bf ? BK * 32 * 2 : 0);
  q.o_wmu = take((q.coop || q.fused) ? BK * q.DP * 2 : 0);
  q.o_wsc = take((q.coop || q.fused) ? BK * 4 : 0);
  q.o_waugs = take(q.fused ? BK * 16 * 2 : 0);
  q.o_cconst = take(BK * 16);
  q.o_covs_used = take(q.cov == SPH ? BK * 4 : (q.cov == DIAG ? BK * q.D * 4 : 0));
  q.o_rowq = take(q.cov == TIED ? BN * 4 : 0);
  q.o_lse2 = take(BN * 4);
  q.o_rowaux = take(sph_bf && q.DP >= 128 ? BN * 16 : 0);
  q.o_pms = take((size_t)std::max(q.ktiles, q.lktiles) * BN * 8);
  q.o_pidx = take((size_t)q.ktiles * BN * 4);
  // (the full-covariance kernels at D > 16 use their own slices only)
  q.o_pstats = take((size_t)(q.fw ? q.fw_slices : std::max({q.slices, q.fslices, q.cspb, q.xslices})) * BK * q.JP * 4);
  q.o_stats = take(BK * q.JP * 4);
  // (+B: the tied EM iteration's per-batch log-likelihood shift, after the row partials)
  q.o_ll = take((size_t)q.B * (std::max({q.cblocks, q.fslices, q.cspb, q.slices, q.xslices, q.fw_eblk}) + q.D + 1) * 8);
  q.o_xch = take(q.coop ? (size_t)q.cNG * kRing * q.cG * kBN * 8
                        : (q.xch ? (size_t)q.B * q.xslices * kRing * q.ktiles * kBN * 8 : 0));
  // [0] status of the last cooperative pass (zeroed by its launcher), [1] sticky
  // status since the last gmmxx_hip_take_status
  q.o_flags = take(8);
  q.o_first = take((size_t)q.chol_m * 4 + 4);   // per-matrix first levels, then the global level
  q.o_lbuf = take(q.chol_m ? (size_t)q.chol_m * chol_dp(q.D) * chol_dp(q.D) * 4 : 0);
  q.o_prec = take(q.fw ? 0 : (size_t)q.chol_m * q.D * q.D * 4);
  q.o_logdet = take((size_t)q.chol_m * 4);
  q.o_gram = take(q.cov == TIED ? (size_t)q.gram_slices * q.B * q.D * q.D * 4 : 0);
  q.o_lpack = take(q.fw ? (size_t)fw_lpack_bytes(q.B, q.K, q.DP) : 0);
  q.o_lpaug = take(q.fw ? BK * (q.DP / 32) * 64 * 8 * 2 : 0);
  q.o_l2w = take(q.fw ? BK * (size_t)q.N * 4 : 0);
  q.o_linv = take((q.fw || q.w16) ? BK * q.D * q.D * 4 : 0);
  q.o_w16parts = take(q.w16 ? BK * 3 * 512 * 2 : 0);   // three 1 KB MFMA operands per component
  q.o_w16b = take(q.w16 ? BK * 16 * 4 : 0);
  q.o_w16c = take(q.w16 ? BK * 4 : 0);
  q.total = off;
  return GMMXX_OK;
}

template <typename T>
T* at(void* ws, size_t off) { return reinterpret_cast<T*>(reinterpret_cast<char*>(ws) + off); }

int check_ws(const Plan& pl, void* ws, int64_t bytes) {
  if (!ws) return fail(GMMXX_ERR_WORKSPACE, "workspace is NULL");
  if (bytes < 0 || (uint64_t)bytes < pl.total)
    return fail(GMMXX_ERR_WORKSPACE, "workspace too small: need " + std::to_string(pl.total) + " bytes");
  if ((uintptr_t)ws % 256 != 0) return fail(GMMXX_ERR_WORKSPACE, "workspace must be 256-byte aligned");
  return GMMXX_OK;
}

int check_hip(const char* what) {
  const hipError_t e = hipGetLastError();
  if (e != hipSuccess) return fail(GMMXX_ERR_HIP, std::string(what) + ": " + hipGetErrorString(e));
  return GMMXX_OK;
}

// em: the EM iteration's passes, whose tied logits leave out the per-row xᵀPx
// (a row constant: responsibilities and labels do not depend on it, and the
// log-likelihood takes it back as -½ tr(P XᵀX) in the combine phase).
TileArgs tile_args(const Plan& pl, const void* x, void* ws, bool em = false) {
  TileArgs a{};
  a.x = x;
  a.vec_ok = (pl.D == pl.DP) && ((uintptr_t)x % 16 == 0);
  a.N = pl.N;
  a.D = pl.D;
  a.K = pl.K;
  a.B = pl.B;
  a.ktiles = pl.ktiles;
  a.rows_per_slice = pl.rows_per_slice;
  a.w_hi = at<void>(ws, pl.o_whi);
  a.w_lo = pl.bf ? at<void>(ws, pl.o_wlo) : nullptr;
  a.w_aug = (pl.bf && pl.cov == SPH) ? at<void>(ws, pl.o_waug) : nullptr;
  a.w_mu = pl.fused ? at<void>(ws, pl.o_wmu) : nullptr;
  a.w_scale = pl.fused ? at<float>(ws, pl.o_wsc) : nullptr;
  a.w_augs = pl.fused ? at<void>(ws, pl.o_waugs) : nullptr;
  a.cconst = at<float4>(ws, pl.o_cconst);
  a.rowq = (pl.cov == TIED && !em) ? at<float>(ws, pl.o_rowq) : nullptr;
  a.lse2 = at<float>(ws, pl.o_lse2);
  a.rowaux = (pl.bf && pl.cov == SPH && pl.DP >= 128) ? at<uint4>(ws, pl.o_rowaux) : nullptr;
  a.part_ms = at<float>(ws, pl.o_pms);
  a.part_idx = at<int>(ws, pl.o_pidx);
  a.part_stats = at<float>(ws, pl.o_pstats);
  a.proba = nullptr;
  a.nslices = pl.fslices;
  a.ll_part = at<double>(ws, pl.o_ll);
  return a;
}

// Launches the tile kernel of `mode` over the plan's grid.
int run_tile(const Plan& pl, int mode, const TileArgs& t, hipStream_t s) {
  if (pl.bf && pl.cov == SPH) {
    TileArgs u = t;
    u.ktiles = mode == MODE_LSE ? pl.lktiles : pl.ktiles;
    return launch_sph_bf16(pl.DP, mode == MODE_LSE ? pl.lnw : pl.nw, mode, u, dim3(pl.slices * u.ktiles, pl.B), s);
  }
  const dim3 grid(pl.slices * pl.ktiles, pl.B);
  return launch_tile(pl.cov, pl.bf, pl.DP, mode, t, grid, pl.nw, s);
}

// Fused pass: partial statistics per row slice and partial log-likelihoods.
int run_fused(const Plan& pl, const TileArgs& t, hipStream_t s) {
  TileArgs u = t;
  u.rows_per_slice = pl.frows;
  return launch_sph_bf16_fused(pl.DP, pl.K, u, pl.fslices, s);
}
// Cooperative single pass: partial statistics per row item and partial log-likelihoods.
int run_coop(const Plan& pl, const void* x, void* ws, hipStream_t s) {
  if ((uintptr_t)x % 16 != 0)
    return fail(GMMXX_ERR_INVALID_ARGUMENT, "x must be 16-byte aligned for spherical bf16 at D = 128");
  CoopArgs c{};
  c.x = x;
  c.vec_ok = 1;
  c.N = pl.N;
  c.D = pl.D;
  c.K = pl.K;
  c.B = pl.B;
  c.w_mu = at<void>(ws, pl.o_wmu);
  c.w_scale = at<float>(ws, pl.o_wsc);
  c.w_aug = at<void>(ws, pl.o_waug);
  c.G = pl.cG;
  c.NG = pl.cNG;
  c.spb = pl.cspb;
  c.rows_per_item = pl.crows;
  c.part_stats = at<float>(ws, pl.o_pstats);
  c.ll_part = at<double>(ws, pl.o_ll);
  c.xch = at<uint64_t>(ws, pl.o_xch);
  c.status = at<unsigned>(ws, pl.o_flags);
  // Polls per wait before the pass gives up; GMMXX_HIP_COOP_SPIN_LIMIT overrides
  // it (a negative value gives up at the first wait: the timeout path, on demand).
  c.spin_limit = 1 << 20;
  if (const char* sl = getenv("GMMXX_HIP_COOP_SPIN_LIMIT")) c.spin_limit = atoi(sl);
  const int rc = launch_sph_bf16_coop(pl.DP, c, s);
  if (rc == -2) return fail(GMMXX_ERR_HIP, "launch of the single-pass cooperative kernel failed");
  if (rc != 0) return fail(GMMXX_ERR_UNSUPPORTED, "no single-pass cooperative kernel for this shape and device");
  return check_hip("cooperative single-pass kernel");
}
// Exchange single pass: partial statistics per row slice and partial log-likelihoods.
// em: the EM iteration's pass (tied logits without the row forms, as tile_args).
int run_xch(const Plan& pl, const void* x, void* ws, hipStream_t s, bool em = true) {
  TileArgs t = tile_args(pl, x, ws, em);
  t.rows_per_slice = pl.xrows;
  t.xch = at<uint64_t>(ws, pl.o_xch);
  t.status = at<unsigned>(ws, pl.o_flags);
  t.spin_limit = 1 << 20;   // as the cooperative pass (GMMXX_HIP_COOP_SPIN_LIMIT overrides)
  if (const char* sl = getenv("GMMXX_HIP_COOP_SPIN_LIMIT")) t.spin_limit = atoi(sl);
  const int64_t nwords = (int64_t)pl.B * pl.xslices * kRing * pl.ktiles * kBN;
  const int rc = launch_tile_xch(pl.cov, pl.DP, t, dim3(pl.xslices * pl.ktiles, pl.B), nwords, s);
  if (rc == -2) return fail(GMMXX_ERR_HIP, "launch of the exchange pass failed");
  if (rc != 0) return fail(GMMXX_ERR_UNSUPPORTED, "no exchange tile kernel for this shape and device");
  return check_hip("exchange single-pass kernel");
}
const unsigned* coop_status(const Plan& pl, void* ws) { return at<unsigned>(ws, pl.o_flags); }
bool single_pass(const Plan& pl) { return pl.fused || pl.coop || pl.single || pl.xch; }
unsigned* sticky_status(const Plan& pl, void* ws) { return at<unsigned>(ws, pl.o_flags) + 1; }
// The log-likelihood sum of a single pass, folded into the slice reduction;
// cooperative and exchange passes also carry their status (a timed-out wait
// makes the value NaN and is added to the sticky word).
LlFold ll_fold(const Plan& pl, void* ws, int parts, double inv_total, float* out) {
  LlFold ll{};
  ll.part = at<double>(ws, pl.o_ll);
  ll.count = parts;
  ll.inv_total = inv_total;
  ll.out = out;
  if (pl.coop || pl.xch) {
    ll.status = at<unsigned>(ws, pl.o_flags);
    ll.sticky = at<unsigned>(ws, pl.o_flags) + 1;
  }
  return ll;
}
int stat_slices(const Plan& pl) {
  return pl.fw ? pl.fw_slices : (pl.fused ? pl.fparts : (pl.coop ? pl.cspb : (pl.xch ? pl.xslices : pl.slices)));
}
// The tile-partial buffer is free once the statistics are being reduced: it is
// the scratch of the grouped slice reduction.
float* red_tmp(const Plan& pl, void* ws) { return at<float>(ws, pl.o_pms); }
int64_t red_tmp_floats(const Plan& pl) { return (int64_t)std::max(pl.ktiles, pl.lktiles) * pl.B * pl.N * 2; }
int ll_parts(const Plan& pl) {
  return pl.B * (pl.fw ? pl.fw_eblk
                       : (pl.fused ? pl.fparts
                                   : (pl.coop ? pl.cspb : (pl.xch ? pl.xslices : (pl.single ? pl.slices : pl.cblocks)))));
}
// The log-likelihood partials come out of the pass itself (no combine phase).
bool ll_in_pass(const Plan& pl) { return single_pass(pl) || pl.fw; }

// Full covariance at D > 16: the E-step / statistics kernels' arguments.
FwArgs fw_args(const Plan& pl, const void* x, void* ws) {
  FwArgs a{};
  a.x = reinterpret_cast<const float*>(x);
  a.vec_ok = (pl.D == pl.DP) && ((uintptr_t)x % 16 == 0);
  a.N = pl.N;
  a.D = pl.D;
  a.K = pl.K;
  a.B = pl.B;
  a.lpack = at<void>(ws, pl.o_lpack);
  a.lpaug = at<void>(ws, pl.o_lpaug);
  a.cconst = at<float4>(ws, pl.o_cconst);
  a.l2 = at<float>(ws, pl.o_l2w);
  a.lse2 = at<float>(ws, pl.o_lse2);
  a.ll_part = at<double>(ws, pl.o_ll);
  a.part_stats = at<float>(ws, pl.o_pstats);
  a.JP = pl.JP;
  a.nk_col = pl.nk_col;
  a.rows_per_slice = pl.fw_rows;
  return a;
}
// Full covariance at D <= 16, K <= 32, inference: Cholesky (L^-1 and log det at the
// batch jitter level), operand packing, then one pass for scores / labels / proba.
int run_w16(const Plan& pl, const void* x, const float* means, const float* covs, const float* weights, void* ws,
            float* scores, int64_t* labels, float* proba, hipStream_t s) {
  launch_chol(covs, pl.D, pl.chol_m, at<int>(ws, pl.o_first), at<int>(ws, pl.o_first) + pl.chol_m,
              at<float>(ws, pl.o_lbuf), nullptr, at<float>(ws, pl.o_logdet), s, at<float>(ws, pl.o_linv));
  Full16Args a{};
  a.x = reinterpret_cast<const float*>(x);
  a.vec_ok = pl.D == 16 && (uintptr_t)x % 16 == 0;
  a.N = pl.N;
  a.D = pl.D;
  a.K = pl.K;
  a.B = pl.B;
  a.linv = at<float>(ws, pl.o_linv);
  a.means = means;
  a.weights = weights;
  a.logdet = at<float>(ws, pl.o_logdet);
  a.lparts = at<void>(ws, pl.o_w16parts);
  a.bneg = at<float>(ws, pl.o_w16b);
  a.c2 = at<float>(ws, pl.o_w16c);
  a.scores = scores;
  a.labels = labels;
  a.proba = proba;
  launch_full16_pack(a, s);
  launch_full16_infer(a, s);
  return check_hip("full-covariance inference");
}

int run_fw(const Plan& pl, int phase, const FwArgs& a, hipStream_t s) {
  if (launch_fw(pl.DP, phase, a, pl.fw_slices, s) != 0) return fail(GMMXX_ERR_UNSUPPORTED, "no full-covariance kernel for this D");
  return check_hip(phase == 0 ? "full-covariance E-step" : "full-covariance statistics");
}
// Where an EM iteration's tied -½ tr(P XᵀX) terms go: after the log-likelihood
// partials of its log-normaliser pass (the single-pass or the combine kernel's),
// so the one reduction sums both; null where no pass leaves the row forms out.
double* tied_shift(const Plan& pl, void* ws) {
  if (pl.cov != TIED || pl.fused || pl.coop) return nullptr;
  return at<double>(ws, pl.o_ll) + ((pl.single || pl.xch) ? ll_parts(pl) : pl.B * pl.cblocks);
}

// Prelude / parameter packing, Cholesky (tied, full) and the tied row forms.
// gram/shift (tied EM without the row forms): the parameter packing also writes
// the -½ tr(P XᵀX) terms, D per problem, to shift.
int prepare(const Plan& pl, const void* x, const float* means, const float* covs, const float* weights,
            double reg, double minw, int prelude, void* ws, hipStream_t s, bool rowquad = true,
            const float* gram = nullptr, double* shift = nullptr) {
  float* prec = nullptr;
  float* logdet = nullptr;
  if (pl.cov == TIED || pl.cov == FULL) {
    prec = at<float>(ws, pl.o_prec);
    logdet = at<float>(ws, pl.o_logdet);
    launch_chol(covs, pl.D, pl.chol_m, at<int>(ws, pl.o_first), at<int>(ws, pl.o_first) + pl.chol_m,
                at<float>(ws, pl.o_lbuf), pl.fw ? nullptr : prec, logdet, s,
                pl.fw ? at<float>(ws, pl.o_linv) : nullptr);
  }
  if (pl.fw) {
    FwPackArgs f{};
    f.B = pl.B;
    f.K = pl.K;
    f.D = pl.D;
    f.DP = pl.DP;
    f.prelude = prelude;
    f.param_round = prelude ? pl.pdt : 0;
    f.min_weight = (float)minw;
    f.means = means;
    f.weights = weights;
    f.linv = at<float>(ws, pl.o_linv);
    f.logdet = logdet;
    f.lpack = at<void>(ws, pl.o_lpack);
    f.lpaug = at<void>(ws, pl.o_lpaug);
    f.cconst = at<float4>(ws, pl.o_cconst);
    launch_fw_pack(f, s);
    return check_hip("parameter preparation");
  }
  PrepArgs a{};
  a.cov = pl.cov;
  a.bf = pl.bf;
  a.prelude = prelude;
  a.param_round = prelude ? pl.pdt : 0;
  a.B = pl.B;
  a.K = pl.K;
  a.D = pl.D;
  a.DP = pl.DP;
  a.EP = pl.EP;
  a.reg_covar = (float)reg;
  a.min_weight = (float)minw;
  a.means = means;
  a.covs = covs;
  a.weights = weights;
  a.prec = prec;
  a.first_ok = (pl.cov == FULL) ? at<int>(ws, pl.o_first) : nullptr;
  a.chol_level = (pl.cov == FULL) ? at<int>(ws, pl.o_first) + pl.chol_m : nullptr;
  a.logdet = logdet;
  a.covs_used = (pl.cov == SPH || pl.cov == DIAG) ? at<float>(ws, pl.o_covs_used) : nullptr;
  a.w_hi = at<void>(ws, pl.o_whi);
  a.w_lo = pl.bf ? at<void>(ws, pl.o_wlo) : nullptr;
  a.w_aug = (pl.bf && pl.cov == SPH) ? at<void>(ws, pl.o_waug) : nullptr;
  a.w_mu = (pl.coop || pl.fused) ? at<void>(ws, pl.o_wmu) : nullptr;
  a.w_scale = (pl.coop || pl.fused) ? at<float>(ws, pl.o_wsc) : nullptr;
  a.w_augs = pl.fused ? at<void>(ws, pl.o_waugs) : nullptr;
  a.cconst = at<float4>(ws, pl.o_cconst);
  a.gram = shift ? gram : nullptr;
  a.shift = gram ? shift : nullptr;
  launch_prep(a, s);
  if (pl.cov == TIED && rowquad)
    launch_rowquad(reinterpret_cast<const float*>(x), pl.B, pl.N, pl.D, prec, at<float>(ws, pl.o_rowq), s);
  return check_hip("parameter preparation");
}

// Log-normaliser pass: per-k-tile partials, then the per-row combine.
int lse_pass(const Plan& pl, const void* x, void* ws, float* scores, int64_t* labels, bool with_ll,
             hipStream_t s) {
  const TileArgs t = tile_args(pl, x, ws);
  if (run_tile(pl, labels ? MODE_LSE_IDX : MODE_LSE, t, s) != 0)
    return fail(GMMXX_ERR_UNSUPPORTED, "no tile kernel for this shape");
  CombineArgs c{};
  c.B = pl.B;
  c.ktiles = labels ? pl.ktiles : pl.lktiles;
  c.N = pl.N;
  c.part_ms = t.part_ms;
  c.part_idx = t.part_idx;
  c.lse2 = at<float>(ws, pl.o_lse2);
  c.scores = scores;
  c.labels = labels;
  c.ll_part = with_ll ? at<double>(ws, pl.o_ll) : nullptr;
  launch_combine(c, s);
  return check_hip("log-normaliser pass");
}

int stats_pass(const Plan& pl, const void* x, void* ws, hipStream_t s) {
  const TileArgs t = tile_args(pl, x, ws);
  if (run_tile(pl, MODE_STATS, t, s) != 0)
    return fail(GMMXX_ERR_UNSUPPORTED, "no tile kernel for this shape");
  launch_reduce_slices(t.part_stats, pl.slices, (int64_t)pl.B * pl.K * pl.JP, at<float>(ws, pl.o_stats), s,
                       red_tmp(pl, ws), red_tmp_floats(pl));
  return check_hip("statistics pass");
}

// M-step parameter update from the statistics rows in the workspace; n_rows is
// the row count per batch that divides N_k into the weights.
// skip: a nonzero word there leaves the parameters unchanged (a timed-out
// cooperative pass), or null.
FinalizeArgs finalize_args(const Plan& pl, void* ws, const float* gram, double reg_covar, double min_weight,
                           int64_t n_rows, float* means, float* covs, float* weights, const unsigned* skip) {
  FinalizeArgs f{};
  f.cov = pl.cov;
  f.B = pl.B;
  f.K = pl.K;
  f.D = pl.D;
  f.DP = pl.DP;
  f.JP = pl.JP;
  f.nk_col = pl.nk_col;
  f.sq_col = pl.sq_col;
  f.sq_n = pl.sq_n;
  f.N = n_rows;
  f.reg_covar = (float)reg_covar;
  f.min_weight = (float)min_weight;
  f.stats = at<float>(ws, pl.o_stats);
  f.covs_used = (pl.cov == SPH || pl.cov == DIAG) ? at<float>(ws, pl.o_covs_used) : nullptr;
  f.gram = gram;
  f.means = means;
  f.covs = covs;
  f.weights = weights;
  f.skip = skip;
  f.bf_means = pl.bf && pl.cov == SPH;
  f.param_round = pl.pdt;
  return f;
}

void finalize(const Plan& pl, void* ws, const float* gram, double reg_covar, double min_weight, int64_t n_rows,
              float* means, float* covs, float* weights, hipStream_t s, const unsigned* skip = nullptr) {
  launch_finalize(finalize_args(pl, ws, gram, reg_covar, min_weight, n_rows, means, covs, weights, skip), s);
}

// Approximate top-k EM: each row's threshold logit and index, per-block
// log-likelihood sums, and (top_k > 1) the (B, N, K) log2 logits, after the
// plan's workspace.  top_k = 1 stops before the logits (`hard`).
struct TopkLayout {
  size_t o_logits = 0, o_thr = 0, o_thri = 0, o_ll = 0, hard = 0, total = 0;
};
TopkLayout topk_layout(const Plan& pl) {
  TopkLayout t;
  size_t off = pl.total;
  auto take = [&](size_t bytes) {
    const size_t o = off;
    off += (bytes + 255) / 256 * 256;
    return o;
  };
  const size_t BN = (size_t)pl.B * pl.N;
  t.o_thr = take(BN * 4);
  t.o_thri = take(BN * 4);
  t.o_ll = take((size_t)pl.B * topk_select_blocks(pl.N) * 8);
  t.hard = off;
  t.o_logits = take(BN * pl.K * 4);
  t.total = off;
  return t;
}

int begin(const gmmxx_problem* p, Plan* pl, const void* x, void* ws, int64_t ws_bytes) {
  int rc = plan_problem(p, pl);
  if (rc) return rc;
  if (!x) return fail(GMMXX_ERR_INVALID_ARGUMENT, "x is NULL");
  return check_ws(*pl, ws, ws_bytes);
}

// The scratch's device address on the current device (looked up once per device).
int scratch_address(void** out) {
  int dev = 0;
  if (hipGetDevice(&dev) != hipSuccess) return check_hip("hipGetDevice");
  if (dev < 0 || dev >= kMaxDevices) return fail(GMMXX_ERR_UNSUPPORTED, "device index beyond the scratch table");
  std::lock_guard<std::mutex> lock(g_scratch_mu);
  if (!g_scratch_ptr[dev]) {
    void* p = nullptr;
    const hipError_t e = hipGetSymbolAddress(&p, HIP_SYMBOL(scratch));
    if (e != hipSuccess || !p) {
      (void)hipGetLastError();
      return fail(GMMXX_ERR_HIP, std::string("hipGetSymbolAddress(scratch): ") + hipGetErrorString(e));
    }
    g_scratch_ptr[dev] = p;
  }
  *out = g_scratch_ptr[dev];
  return GMMXX_OK;
}

}  // namespace

extern "C" {

int gmmxx_hip_abi_version(void) { return GMMXX_HIP_ABI_VERSION; }

const char* gmmxx_hip_last_error(void) { return g_last_error.c_str(); }

int gmmxx_hip_canary(const int32_t* in, int32_t* out, int64_t n, int32_t offset, void* stream) {
  if (n < 0) return fail(GMMXX_ERR_INVALID_ARGUMENT, "n must be non-negative");
  if (n == 0) return GMMXX_OK;
  if (!in || !out) return fail(GMMXX_ERR_INVALID_ARGUMENT, "NULL buffer");
  launch_canary(in, out, n, offset, (hipStream_t)stream);
  return check_hip("canary");
}

int gmmxx_hip_device_info(int device, gmmxx_dev_info* out) {
  if (!out) return fail(GMMXX_ERR_INVALID_ARGUMENT, "out is NULL");
  int ndev = 0;
  if (hipGetDeviceCount(&ndev) != hipSuccess || device < 0 || device >= ndev) {
    (void)hipGetLastError();
    return fail(GMMXX_ERR_INVALID_ARGUMENT, "no such device");
  }
  hipDeviceProp_t prop;
  if (hipGetDeviceProperties(&prop, device) != hipSuccess) return check_hip("hipGetDeviceProperties");
  *out = gmmxx_dev_info{};
  out->device = device;
  snprintf(out->arch, sizeof(out->arch), "%s", prop.gcnArchName);
  out->supported = strncmp(prop.gcnArchName, "gfx950", 6) == 0 ? 1 : 0;
  out->compute_units = prop.multiProcessorCount;
  out->wave_size = prop.warpSize;
  out->clock_khz = prop.clockRate;
  out->hbm_bytes = (int64_t)prop.totalGlobalMem;
  out->lds_per_workgroup = (int64_t)prop.sharedMemPerBlock;
  int cur = 0;
  if (hipGetDevice(&cur) != hipSuccess) return check_hip("hipGetDevice");
  if (cur != device && hipSetDevice(device) != hipSuccess) return check_hip("hipSetDevice");
  out->coop_capacity = coop_capacity();
  if (cur != device && hipSetDevice(cur) != hipSuccess) return check_hip("hipSetDevice");
  return GMMXX_OK;
}

int gmmxx_hip_supported(const gmmxx_problem* p) {
  Plan pl;
  const std::string saved = g_last_error;
  const int rc = plan_problem(p, &pl);
  g_last_error = saved;
  return rc == GMMXX_OK ? 1 : 0;
}

int64_t gmmxx_hip_workspace_bytes(const gmmxx_problem* p) {
  Plan pl;
  if (plan_problem(p, &pl) != GMMXX_OK) return -1;
  return (int64_t)pl.total;
}

int gmmxx_hip_take_status(const gmmxx_problem* p, void* ws, int64_t ws_bytes, uint32_t* status_out,
                          void* stream) {
  Plan pl;
  int rc = plan_problem(p, &pl);
  if (rc) return rc;
  if ((rc = check_ws(pl, ws, ws_bytes))) return rc;
  if (!status_out) return fail(GMMXX_ERR_INVALID_ARGUMENT, "status_out is NULL");
  launch_take_status(sticky_status(pl, ws), status_out, (hipStream_t)stream);
  return check_hip("take_status");
}

int gmmxx_hip_em_phase(const gmmxx_problem* p, int phase, const void* x, float* means, float* covs,
                       float* weights, const float* gram, double reg_covar, double min_weight,
                       float* lower_bound, void* ws, int64_t ws_bytes, void* stream) {
  Plan pl;
  int rc = begin(p, &pl, x, ws, ws_bytes);
  if (rc) return rc;
  if (!means || !covs || !weights || !lower_bound) return fail(GMMXX_ERR_INVALID_ARGUMENT, "NULL parameter buffer");
  if (pl.cov == TIED && !gram) return fail(GMMXX_ERR_INVALID_ARGUMENT, "tied EM needs the XᵀX buffer");
  if (!(min_weight > 0.0)) return fail(GMMXX_ERR_INVALID_ARGUMENT, "min_weight must be positive");
  const hipStream_t s = (hipStream_t)stream;
  switch (phase) {
    case GMMXX_PHASE_PREPARE:
      return prepare(pl, x, means, covs, weights, reg_covar, min_weight, 1, ws, s, /*rowquad=*/false, gram,
                     tied_shift(pl, ws));
    case GMMXX_PHASE_LSE_TILE: {
      if (pl.fw) return run_fw(pl, 0, fw_args(pl, x, ws), s);
      if (pl.coop) return run_coop(pl, x, ws, s);
      if (pl.xch) return run_xch(pl, x, ws, s, /*em=*/true);
      const TileArgs t = tile_args(pl, x, ws, /*em=*/true);
      if (pl.single) {
        if (run_tile(pl, MODE_STATS_LSE, t, s) != 0) return fail(GMMXX_ERR_UNSUPPORTED, "no tile kernel for this shape");
        return check_hip("single-pass tile kernel");
      }
      if ((pl.fused ? run_fused(pl, t, s) : run_tile(pl, MODE_LSE, t, s)) != 0)
        return fail(GMMXX_ERR_UNSUPPORTED, "no tile kernel for this shape");
      return check_hip(pl.fused ? "fused tile kernel" : "log-normaliser tile kernel");
    }
    case GMMXX_PHASE_COMBINE: {
      // A single pass already produced per-slice log-likelihoods: they are summed
      // by the reduce phase's launch (one launch fewer per iteration).
      if (ll_in_pass(pl)) return GMMXX_OK;
      CombineArgs c{};
      c.B = pl.B;
      c.ktiles = pl.lktiles;
      c.N = pl.N;
      c.part_ms = at<float>(ws, pl.o_pms);
      c.part_idx = at<int>(ws, pl.o_pidx);
      c.lse2 = at<float>(ws, pl.o_lse2);
      c.ll_part = at<double>(ws, pl.o_ll);
      launch_combine(c, s);
      int parts = pl.B * pl.cblocks;
      if (tied_shift(pl, ws)) parts += pl.B * pl.D;   // -½ tr(P XᵀX) rows, from the prepare phase
      launch_ll_reduce(at<double>(ws, pl.o_ll), parts, 1.0 / ((double)pl.B * (double)pl.N), lower_bound, s);
      return check_hip("combine");
    }
    case GMMXX_PHASE_STATS_TILE: {
      if (pl.fw) return run_fw(pl, 1, fw_args(pl, x, ws), s);
      if (single_pass(pl)) return GMMXX_OK;  // statistics came out of the single pass
      const TileArgs t = tile_args(pl, x, ws, /*em=*/true);
      if (run_tile(pl, MODE_STATS, t, s) != 0)
        return fail(GMMXX_ERR_UNSUPPORTED, "no tile kernel for this shape");
      return check_hip("statistics tile kernel");
    }
    case GMMXX_PHASE_REDUCE: {
      LlFold ll{};
      if (ll_in_pass(pl)) {
        int parts = ll_parts(pl);
        if (tied_shift(pl, ws)) parts += pl.B * pl.D;   // -½ tr(P XᵀX) rows, from the prepare phase
        ll = ll_fold(pl, ws, parts, 1.0 / ((double)pl.B * (double)pl.N), lower_bound);
      }
      launch_reduce_slices(at<float>(ws, pl.o_pstats), stat_slices(pl), (int64_t)pl.B * pl.K * pl.JP,
                           at<float>(ws, pl.o_stats), s, red_tmp(pl, ws), red_tmp_floats(pl),
                           ll_in_pass(pl) ? &ll : nullptr);
      return check_hip("statistics reduction");
    }
    case GMMXX_PHASE_FINALIZE:
      // A cooperative pass that timed out leaves the parameters as they were.
      finalize(pl, ws, gram, reg_covar, min_weight, pl.N, means, covs, weights, s,
               (pl.coop || pl.xch) ? coop_status(pl, ws) : nullptr);
      return check_hip("finalize");
    default:
      return fail(GMMXX_ERR_INVALID_ARGUMENT, "unknown phase");
  }
}

int gmmxx_hip_em_step(const gmmxx_problem* p, const void* x, float* means, float* covs, float* weights,
                      const float* gram, double reg_covar, double min_weight, float* lower_bound,
                      void* ws, int64_t ws_bytes, void* stream) {
  for (int ph = GMMXX_PHASE_PREPARE; ph <= GMMXX_PHASE_FINALIZE; ++ph) {
    const int rc = gmmxx_hip_em_phase(p, ph, x, means, covs, weights, gram, reg_covar, min_weight,
                                      lower_bound, ws, ws_bytes, stream);
    if (rc) return rc;
  }
  return GMMXX_OK;
}

int gmmxx_hip_em_step_noalloc(const gmmxx_problem* p, const void* x, float* means, float* covs, float* weights,
                              const float* gram, double reg_covar, double min_weight, float* lower_bound,
                              void* stream) {
  Plan pl;
  int rc = plan_problem(p, &pl);
  if (rc) return rc;
  if ((int64_t)pl.total > kScratchBytes)
    return fail(GMMXX_ERR_WORKSPACE, "problem needs " + std::to_string(pl.total) +
                                         " bytes of scratch, above the no-allocation limit of " +
                                         std::to_string(kScratchBytes) + " bytes; use gmmxx_hip_em_step");
  void* ws = nullptr;
  if ((rc = scratch_address(&ws))) return rc;
  // The status words are the only scratch bytes read before a call writes them
  // (the coop launcher zeroes its exchange words itself): clear them with a
  // kernel, which a caller may also capture in a graph.
  launch_zero_words(at<unsigned>(ws, pl.o_flags), 2, (hipStream_t)stream);
  return gmmxx_hip_em_step(p, x, means, covs, weights, gram, reg_covar, min_weight, lower_bound, ws, kScratchBytes,
                           stream);
}

int gmmxx_hip_estep_stats(const gmmxx_problem* p, const void* x, const float* means, const float* covs,
                          const float* weights, double reg_covar, double min_weight, float* nk, float* sum_x,
                          float* sum_q, float* ll_sum, void* ws, int64_t ws_bytes, void* stream) {
  Plan pl;
  int rc = begin(p, &pl, x, ws, ws_bytes);
  if (rc) return rc;
  if (!means || !covs || !weights || !nk || !sum_x || !ll_sum)
    return fail(GMMXX_ERR_INVALID_ARGUMENT, "NULL buffer");
  if (pl.cov != TIED && !sum_q) return fail(GMMXX_ERR_INVALID_ARGUMENT, "sum_q is required for this covariance type");
  if (!(min_weight > 0.0)) return fail(GMMXX_ERR_INVALID_ARGUMENT, "min_weight must be positive");
  const hipStream_t s = (hipStream_t)stream;
  if ((rc = prepare(pl, x, means, covs, weights, reg_covar, min_weight, 1, ws, s))) return rc;
  if (pl.fw) {
    const FwArgs a = fw_args(pl, x, ws);
    if ((rc = run_fw(pl, 0, a, s)) || (rc = run_fw(pl, 1, a, s))) return rc;
    const LlFold ll = ll_fold(pl, ws, ll_parts(pl), 1.0, ll_sum);
    launch_reduce_slices(at<float>(ws, pl.o_pstats), stat_slices(pl), (int64_t)pl.B * pl.K * pl.JP,
                         at<float>(ws, pl.o_stats), s, red_tmp(pl, ws), red_tmp_floats(pl), &ll);
    if ((rc = check_hip("full-covariance statistics reduction"))) return rc;
  } else if (pl.fused || pl.coop || pl.single || pl.xch) {
    if (pl.coop) {
      if ((rc = run_coop(pl, x, ws, s))) return rc;
    } else if (pl.xch) {
      if ((rc = run_xch(pl, x, ws, s, /*em=*/false))) return rc;
    } else if (pl.single) {
      if (run_tile(pl, MODE_STATS_LSE, tile_args(pl, x, ws), s) != 0)
        return fail(GMMXX_ERR_UNSUPPORTED, "no tile kernel for this shape");
    } else if (run_fused(pl, tile_args(pl, x, ws), s) != 0) {
      return fail(GMMXX_ERR_UNSUPPORTED, "no fused kernel for this shape");
    }
    const LlFold ll = ll_fold(pl, ws, ll_parts(pl), 1.0, ll_sum);
    launch_reduce_slices(at<float>(ws, pl.o_pstats), stat_slices(pl), (int64_t)pl.B * pl.K * pl.JP,
                         at<float>(ws, pl.o_stats), s, red_tmp(pl, ws), red_tmp_floats(pl), &ll);
    if ((rc = check_hip("fused statistics pass"))) return rc;
  } else {
    if ((rc = lse_pass(pl, x, ws, nullptr, nullptr, true, s))) return rc;
    launch_ll_reduce(at<double>(ws, pl.o_ll), pl.B * pl.cblocks, 1.0, ll_sum, s);
    if ((rc = stats_pass(pl, x, ws, s))) return rc;
  }
  UnpackArgs u{};
  u.cov = pl.cov;
  u.K = pl.K;
  u.D = pl.D;
  u.DP = pl.DP;
  u.JP = pl.JP;
  u.nk_col = pl.nk_col;
  u.sq_col = pl.sq_col;
  u.sq_n = pl.sq_n;
  u.stats = at<float>(ws, pl.o_stats);
  u.nk = nk;
  u.sum_x = sum_x;
  u.sum_q = pl.cov == TIED ? nullptr : sum_q;
  launch_unpack(u, pl.B, s);
  return check_hip("statistics unpack");
}

int64_t gmmxx_hip_topk_workspace_bytes(const gmmxx_problem* p, int top_k) {
  Plan pl;
  if (plan_problem(p, &pl) != GMMXX_OK) return -1;
  const TopkLayout tl = topk_layout(pl);
  return (int64_t)(top_k == 1 ? tl.hard : tl.total);
}

int gmmxx_hip_estep_stats_topk(const gmmxx_problem* p, const void* x, const float* means, const float* covs,
                               const float* weights, double reg_covar, double min_weight, int top_k, float* nk,
                               float* sum_x, float* sum_q, float* ll_sum, void* ws, int64_t ws_bytes,
                               void* stream) {
  Plan pl;
  int rc = plan_problem(p, &pl);
  if (rc) return rc;
  if (!x) return fail(GMMXX_ERR_INVALID_ARGUMENT, "x is NULL");
  const TopkLayout tl = topk_layout(pl);
  const size_t need = top_k == 1 ? tl.hard : tl.total;
  if (!ws) return fail(GMMXX_ERR_WORKSPACE, "workspace is NULL");
  if (ws_bytes < 0 || (uint64_t)ws_bytes < need)
    return fail(GMMXX_ERR_WORKSPACE, "workspace too small: need " + std::to_string(need) + " bytes");
  if ((uintptr_t)ws % 256 != 0) return fail(GMMXX_ERR_WORKSPACE, "workspace must be 256-byte aligned");
  if (!means || !covs || !weights || !nk || !sum_x || !ll_sum) return fail(GMMXX_ERR_INVALID_ARGUMENT, "NULL buffer");
  if (pl.cov != TIED && !sum_q) return fail(GMMXX_ERR_INVALID_ARGUMENT, "sum_q is required for this covariance type");
  if (!(min_weight > 0.0)) return fail(GMMXX_ERR_INVALID_ARGUMENT, "min_weight must be positive");
  if (top_k < 1 || top_k >= pl.K)
    return fail(GMMXX_ERR_INVALID_ARGUMENT, "top_k must be in [1, K-1] (top_k >= K is exact EM)");
  const hipStream_t s = (hipStream_t)stream;
  // Parameters with the iteration prelude; tied rows get xᵀPx, so the logits
  // (and the log-normalisers) are complete.
  if ((rc = prepare(pl, x, means, covs, weights, reg_covar, min_weight, 1, ws, s))) return rc;
  // spherical bf16 at D = 128: the later passes read the augmented row chunk
  // that the log-normaliser pass stores.
  float* thr = at<float>(ws, tl.o_thr);
  int* thri = at<int>(ws, tl.o_thri);
  if (pl.fw && top_k == 1) {
    // hard assignment: first argmax per row, then the one-hot statistics
    FwArgs a = fw_args(pl, x, ws);
    a.l2 = nullptr;
    a.hard = 1;
    a.hard_idx = thri;
    a.lse2 = thr;
    if ((rc = run_fw(pl, 0, a, s)) || (rc = run_fw(pl, 1, a, s))) return rc;
    const LlFold ll = ll_fold(pl, ws, ll_parts(pl), 1.0, ll_sum);
    launch_reduce_slices(at<float>(ws, pl.o_pstats), stat_slices(pl), (int64_t)pl.B * pl.K * pl.JP,
                         at<float>(ws, pl.o_stats), s, red_tmp(pl, ws), red_tmp_floats(pl), &ll);
  } else if (pl.fw) {
    // the E-step's (B, K, N) log2 logits, transposed to (B, N, K) for the per-row
    // top-k selection (threshold, index, top-k log-normaliser), then the statistics
    // over each row's kept components
    FwArgs a = fw_args(pl, x, ws);
    a.ll_part = nullptr;
    if ((rc = run_fw(pl, 0, a, s))) return rc;
    float* logits = at<float>(ws, tl.o_logits);
    launch_fw_proba(a.l2, a.lse2, logits, pl.B, pl.N, pl.K, s, /*raw=*/true);
    double* tll = at<double>(ws, tl.o_ll);
    const int sel_blocks = topk_select_blocks(pl.N);
    launch_topk_select(logits, pl.B, pl.N, pl.K, top_k, a.lse2, thr, thri, tll, sel_blocks, s);
    a.thr2 = thr;
    a.thr_idx = thri;
    if ((rc = run_fw(pl, 1, a, s))) return rc;
    launch_reduce_slices(at<float>(ws, pl.o_pstats), stat_slices(pl), (int64_t)pl.B * pl.K * pl.JP,
                         at<float>(ws, pl.o_stats), s, red_tmp(pl, ws), red_tmp_floats(pl));
    launch_ll_reduce(tll, pl.B * sel_blocks, 1.0, ll_sum, s);
  } else if (top_k == 1) {
    // Hard assignment: the first-argmax pass gives each row's maximum (the
    // log-normaliser of a single component) and its index; the statistics pass
    // then gives that component r = 1 by index, no logits stored.
    TileArgs t = tile_args(pl, x, ws);
    if (run_tile(pl, MODE_LSE_IDX, t, s) != 0) return fail(GMMXX_ERR_UNSUPPORTED, "no tile kernel for this shape");
    CombineArgs c{};
    c.B = pl.B;
    c.ktiles = pl.ktiles;
    c.N = pl.N;
    c.part_ms = t.part_ms;
    c.part_idx = t.part_idx;
    c.lse2 = thr;
    c.idx32 = thri;
    c.max_only = 1;
    c.ll_part = at<double>(ws, pl.o_ll);
    launch_combine(c, s);
    TileArgs u = tile_args(pl, x, ws);
    u.lse2 = thr;
    u.thr2 = thr;
    u.thr_idx = thri;
    u.hard = 1;
    if (run_tile(pl, MODE_STATS_TOPK, u, s) != 0) return fail(GMMXX_ERR_UNSUPPORTED, "no tile kernel for this shape");
    launch_reduce_slices(u.part_stats, pl.slices, (int64_t)pl.B * pl.K * pl.JP, at<float>(ws, pl.o_stats), s,
                         red_tmp(pl, ws), red_tmp_floats(pl));
    launch_ll_reduce(at<double>(ws, pl.o_ll), pl.B * pl.cblocks, 1.0, ll_sum, s);
  } else {
  if (pl.bf && pl.cov == SPH && pl.DP >= 128) {
    if ((rc = lse_pass(pl, x, ws, nullptr, nullptr, false, s))) return rc;
  }
  float* logits = at<float>(ws, tl.o_logits);
  double* tll = at<double>(ws, tl.o_ll);
  TileArgs t = tile_args(pl, x, ws);
  t.proba = logits;
  t.raw_logits = 1;
  if (run_tile(pl, MODE_PROBA, t, s) != 0) return fail(GMMXX_ERR_UNSUPPORTED, "no tile kernel for this shape");
  const int sel_blocks = topk_select_blocks(pl.N);
  launch_topk_select(logits, pl.B, pl.N, pl.K, top_k, at<float>(ws, pl.o_lse2), thr, thri, tll, sel_blocks, s);
  TileArgs u = tile_args(pl, x, ws);
  u.thr2 = thr;
  u.thr_idx = thri;
  if (run_tile(pl, MODE_STATS_TOPK, u, s) != 0) return fail(GMMXX_ERR_UNSUPPORTED, "no tile kernel for this shape");
  launch_reduce_slices(u.part_stats, pl.slices, (int64_t)pl.B * pl.K * pl.JP, at<float>(ws, pl.o_stats), s,
                       red_tmp(pl, ws), red_tmp_floats(pl));
  launch_ll_reduce(tll, pl.B * sel_blocks, 1.0, ll_sum, s);
  }
  if ((rc = check_hip("approximate top-k statistics"))) return rc;
  UnpackArgs k{};
  k.cov = pl.cov;
  k.K = pl.K;
  k.D = pl.D;
  k.DP = pl.DP;
  k.JP = pl.JP;
  k.nk_col = pl.nk_col;
  k.sq_col = pl.sq_col;
  k.sq_n = pl.sq_n;
  k.stats = at<float>(ws, pl.o_stats);
  k.nk = nk;
  k.sum_x = sum_x;
  k.sum_q = pl.cov == TIED ? nullptr : sum_q;
  launch_unpack(k, pl.B, s);
  return check_hip("statistics unpack");
}

int gmmxx_hip_finalize_stats(const gmmxx_problem* p, const float* nk, const float* sum_x, const float* sum_q,
                             const float* gram, double reg_covar, double min_weight, float* means, float* covs,
                             float* weights, void* ws, int64_t ws_bytes, void* stream) {
  if (!p) return fail(GMMXX_ERR_INVALID_ARGUMENT, "problem descriptor is NULL");
  gmmxx_problem one = *p;   // the statistics rows do not depend on N: plan for one row
  one.N = 1;
  Plan pl;
  int rc = plan_problem(&one, &pl);
  if (rc) return rc;
  if ((rc = check_ws(pl, ws, ws_bytes))) return rc;
  if (!nk || !sum_x || !means || !covs || !weights) return fail(GMMXX_ERR_INVALID_ARGUMENT, "NULL buffer");
  if (pl.cov != TIED && !sum_q) return fail(GMMXX_ERR_INVALID_ARGUMENT, "sum_q is required for this covariance type");
  if (pl.cov == TIED && !gram) return fail(GMMXX_ERR_INVALID_ARGUMENT, "tied finalize needs the XᵀX buffer");
  if (!(min_weight > 0.0)) return fail(GMMXX_ERR_INVALID_ARGUMENT, "min_weight must be positive");
  const hipStream_t s = (hipStream_t)stream;
  PackArgs k{};
  k.cov = pl.cov;
  k.K = pl.K;
  k.D = pl.D;
  k.DP = pl.DP;
  k.JP = pl.JP;
  k.nk_col = pl.nk_col;
  k.sq_col = pl.sq_col;
  k.reg_covar = (float)reg_covar;
  k.nk = nk;
  k.sum_x = sum_x;
  k.sum_q = sum_q;
  k.covs = covs;
  k.stats = at<float>(ws, pl.o_stats);
  k.covs_used = (pl.cov == SPH || pl.cov == DIAG) ? at<float>(ws, pl.o_covs_used) : nullptr;
  launch_pack(k, pl.B, s);
  finalize(pl, ws, gram, reg_covar, min_weight, p->N, means, covs, weights, s);
  return check_hip("finalize from statistics");
}

int gmmxx_hip_score(const gmmxx_problem* p, const void* x, const float* means, const float* covs,
                    const float* weights, float* scores, int64_t* labels, void* ws, int64_t ws_bytes,
                    void* stream) {
  Plan pl;
  int rc = begin(p, &pl, x, ws, ws_bytes);
  if (rc) return rc;
  if (!means || !covs || !weights) return fail(GMMXX_ERR_INVALID_ARGUMENT, "NULL parameter buffer");
  const hipStream_t s = (hipStream_t)stream;
  if (pl.w16) return run_w16(pl, x, means, covs, weights, ws, scores, labels, nullptr, s);
  if ((rc = prepare(pl, x, means, covs, weights, 0.0, 1e-8, 0, ws, s))) return rc;
  if (pl.fw) {
    FwArgs a = fw_args(pl, x, ws);
    a.l2 = nullptr;
    a.ll_part = nullptr;
    a.scores = scores;
    a.labels = labels;
    return run_fw(pl, 0, a, s);
  }
  return lse_pass(pl, x, ws, scores, labels, false, s);
}

int gmmxx_hip_predict_proba_score(const gmmxx_problem* p, const void* x, const float* means, const float* covs,
                                  const float* weights, float* proba, float* scores, void* ws, int64_t ws_bytes,
                                  void* stream) {
  Plan pl;
  int rc = begin(p, &pl, x, ws, ws_bytes);
  if (rc) return rc;
  if (!means || !covs || !weights) return fail(GMMXX_ERR_INVALID_ARGUMENT, "NULL parameter buffer");
  if (!proba && !scores) return fail(GMMXX_ERR_INVALID_ARGUMENT, "proba and scores are both NULL");
  const hipStream_t s = (hipStream_t)stream;
  if (pl.w16) return run_w16(pl, x, means, covs, weights, ws, scores, nullptr, proba, s);
  if ((rc = prepare(pl, x, means, covs, weights, 0.0, 1e-8, 0, ws, s))) return rc;
  if (pl.fw) {
    FwArgs a = fw_args(pl, x, ws);
    if (!proba) a.l2 = nullptr;
    a.ll_part = nullptr;
    a.scores = scores;
    if ((rc = run_fw(pl, 0, a, s))) return rc;
    if (proba) launch_fw_proba(a.l2, a.lse2, proba, pl.B, pl.N, pl.K, s);
    return check_hip("predict_proba");
  }
  if (!proba) return lse_pass(pl, x, ws, scores, nullptr, false, s);
  // One tile pass when the workgroup holds every component (the pass forms the
  // row log-normalisers, which are the scores); otherwise the log-normaliser
  // pass writes the scores and the responsibility pass reads its lse.
  if (!pl.single && (rc = lse_pass(pl, x, ws, scores, nullptr, false, s))) return rc;
  TileArgs t = tile_args(pl, x, ws);
  t.proba = proba;
  t.scores = pl.single ? scores : nullptr;
  if (run_tile(pl, pl.single ? MODE_PROBA_LSE : MODE_PROBA, t, s) != 0)
    return fail(GMMXX_ERR_UNSUPPORTED, "no tile kernel for this shape");
  return check_hip("predict_proba");
}

int gmmxx_hip_predict_proba(const gmmxx_problem* p, const void* x, const float* means, const float* covs,
                            const float* weights, float* proba, void* ws, int64_t ws_bytes, void* stream) {
  if (!proba) return fail(GMMXX_ERR_INVALID_ARGUMENT, "NULL buffer");
  return gmmxx_hip_predict_proba_score(p, x, means, covs, weights, proba, nullptr, ws, ws_bytes, stream);
}

int gmmxx_hip_gram(const gmmxx_problem* p, const void* x, float* out, void* ws, int64_t ws_bytes, void* stream) {
  Plan pl;
  int rc = begin(p, &pl, x, ws, ws_bytes);
  if (rc) return rc;
  if (pl.cov != TIED) return fail(GMMXX_ERR_INVALID_ARGUMENT, "gram is defined for the tied problem");
  if (!out) return fail(GMMXX_ERR_INVALID_ARGUMENT, "out is NULL");
  const hipStream_t s = (hipStream_t)stream;
  float* part = at<float>(ws, pl.o_gram);
  launch_gram(reinterpret_cast<const float*>(x), pl.B, pl.N, pl.D, pl.gram_slices, pl.gram_rows, part, s);
  launch_reduce_slices(part, pl.gram_slices, (int64_t)pl.B * pl.D * pl.D, out, s);
  return check_hip("gram");
}

int64_t gmmxx_hip_kmeans_pp_workspace_bytes(int64_t B, int64_t S, int64_t D, int64_t K, int trials) {
  if (B < 1 || B > 65535 || S < 1 || S > kKppMaxRows || D < 1 || D > 1024 || K < 1 || K > S || trials < 1 ||
      trials > kKppMaxTrials)
    return -1;
  return kpp_workspace_bytes((int)B, (int)S, (int)K, trials);
}

int gmmxx_hip_kmeans_pp(const float* sample, int64_t B, int64_t S, int64_t D, int64_t K, int trials,
                        const int64_t* first_idx, const float* draws, float* centers, void* ws, int64_t ws_bytes,
                        void* stream) {
  const int64_t need = gmmxx_hip_kmeans_pp_workspace_bytes(B, S, D, K, trials);
  if (need < 0)
    return fail(GMMXX_ERR_INVALID_ARGUMENT,
                "k-means++ needs 1 <= B <= 65535, 1 <= K <= S <= 65536, 1 <= D <= 1024, 1 <= trials <= 16");
  if (!sample || !first_idx || !centers || (K > 1 && !draws)) return fail(GMMXX_ERR_INVALID_ARGUMENT, "NULL buffer");
  if (!ws) return fail(GMMXX_ERR_WORKSPACE, "workspace is NULL");
  if (ws_bytes < need) return fail(GMMXX_ERR_WORKSPACE, "workspace too small: need " + std::to_string(need) + " bytes");
  if ((uintptr_t)ws % 256 != 0) return fail(GMMXX_ERR_WORKSPACE, "workspace must be 256-byte aligned");
  KppArgs a{};
  a.sample = sample;
  a.B = (int)B;
  a.S = (int)S;
  a.D = (int)D;
  a.K = (int)K;
  a.T = trials;
  a.vec = (D % 4 == 0) && ((uintptr_t)sample % 16 == 0);
  a.first = first_idx;
  a.draws = draws;
  a.centers = centers;
  kpp_bind_workspace(a, ws);
  launch_kpp(a, (hipStream_t)stream);
  return check_hip("k-means++ seeding");
}

}  // extern "C"
