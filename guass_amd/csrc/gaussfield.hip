// gaussfield.hip - gfx950 kernels and C ABI of libgaussfield.so.
//
// Forward (reference forward.cu:372-569).  Mask path (16x16 or 32x32 tiles, K <= 8192), three
// kernels:
//   k_prep     four lanes per Gaussian (one thread above 2048 Gaussians): bit-exact sigma-box
//              tile rectangle, fp32 covariance and evaluation constants.
//   k_bin_tiles one workgroup per tile row and per tile column, none waiting for another: the
//              row's or column's bitmask of the Gaussians whose tile range covers it (wave
//              ballots), and per tile row the tile_ptr of its tiles (a closed-form count of
//              the pairs in earlier rows plus a scan of the row's column differences).
//   k_render16 (below).
//   Single 16x16 fields of 257..1024 Gaussians skip k_bin_tiles: k_render16x2_rows bins a tile
//   row per workgroup (the K rectangles tested against the row once, a barrier, the row's
//   Gaussians listed in LDS in id order, each wave's two tiles taken from that list), and
//   k_prep also stores the chain-rule maps.  Up to 256 Gaussians each tile's wave bins itself.
// Emission path, three kernels:
//   k_bin      one workgroup per field: rectangles, the pair total, per-tile Gaussian counts
//              from row-wise difference arrays and their scan -> tile_ptr; every scan runs in
//              LDS (DPP wave scans) and global memory is only written, coalesced.  (The
//              batched form, k_bin_batch, one workgroup per field, also builds the masks.)
//   k_emit     (emission path) one wave per Gaussian: its evaluation constants (kept in the
//              workspace for the render and the backward) and a slot in each touched tile's
//              range from tile_ptr and a per-tile fill counter (a counting sort on the tile key).
//   k_render16 one wave per 16x16 tile (or 16x16 quadrant of a 32x32 tile), four per
//              workgroup, no workgroup barriers: the tile's ids in canonical (ascending gid) order -- the set bits of
//              rowmask & colmask (mask path) or k_emit's segment sorted -- written to the
//              tile's segment, per-Gaussian constants loaded one Gaussian per lane and broadcast
//              with readlane, 4 pixels per lane with per-row terms hoisted.
//   (k_render_any handles other tile shapes.)
// Backward (reference backward.cu:541-716), two kernels:
//   k_bwd16    one wave per 16x16 tile: lanes are (Gaussian slot, tile row); each lane sums
//              16 pixels of its row for its Gaussian into six moments, 16-lane DPP row sums
//              reduce them, and one atomic per (Gaussian, tile, moment) accumulates them.
//   k_bwd_finish  per Gaussian: chain rule from the six moments to (mu, chol_raw, amp), in
//              double, then clears the accumulators so the workspace stays zeroed.
//   (k_bwd_any handles other tile shapes.)
// The quadratic form of a pixel is evaluated in whitened form, q = |R d|^2 with R the inverse
// of the exact Cholesky factor of the fp32 covariance: its fp32 rounding error grows like
// sqrt(cond) instead of cond, which matters for strongly anisotropic Gaussians.
#include <hip/hip_runtime.h>

#include <algorithm>
#include <cmath>
#include <cstdarg>
#include <cstddef>
#include <cstdint>
#include <cstdio>
#include <cstring>
#include <mutex>
#include <type_traits>
#include <vector>

#include "../../include/gaussfield.h"
#include "geometry.h"

#define GF_VERSION "gaussfield-mi355x 0.2.0"

namespace {

constexpr int kBinThreads = 1024;
constexpr int kTileThreads = 256;
constexpr int kEmitThreads = 256;
constexpr int kLdsDiffWords = 12288;  // 48 KiB row-difference band in k_bin
constexpr int kBinMaxBandRows = 1024; // row totals kept in LDS per band in k_bin
constexpr int kMaskLdsWords = 16384;  // 64 KiB band of tile-row / tile-column masks in k_bin
constexpr int kLongSpan = 32;         // k_bin: rectangles spanning more rows / columns than this
constexpr int kLongMax = 256;         //   go to a list of up to kLongMax spread over the workgroup
constexpr int64_t kMaskMaxK = 8192;   // mask path up to this many Gaussians (256 words a mask)
constexpr int64_t kMaskMaxWords = int64_t(1) << 24;  // and up to (R + C) * W mask words

// k_bin counts a tile grid of C columns in LDS bands (int32 row sums) when this holds;
// otherwise through global memory.
__host__ __device__ inline bool bin_counts_in_lds(int64_t C, int64_t K) {
  return (C | 1) <= kLdsDiffWords && K * C < (int64_t)INT32_MAX;
}
constexpr int kSortLdsKeys = 2048;    // (any-shape kernels) segments up to this length in LDS
constexpr int kBitmapMaxK = 131072;   // (any-shape kernels) longer segments: K-bit bitmap
constexpr int kSortLdsWords = (kSortLdsKeys > kBitmapMaxK / 32) ? kSortLdsKeys : kBitmapMaxK / 32;
constexpr int kWaveSortKeys = 512;
constexpr int kHeavyChunk = 16;       // Gaussians per chunk of a heavy tile's four waves    // (16x16 kernels) per-wave LDS keys / bitmap words
// exp(-q/2) = 2^(q * kHalfLog2e); the clamp q in [0, clamp] maps to [clamp * kHalfLog2e, 0].
constexpr float kHalfLog2e = -0.72134752044448170368f;
constexpr double kSqrtHalfLog2e = 0.84932180028801904272;  // sqrt(-kHalfLog2e)

thread_local char g_err[1024];

int set_err(int code, const char* fmt, ...) {
  va_list ap;
  va_start(ap, fmt);
  vsnprintf(g_err, sizeof(g_err), fmt, ap);
  va_end(ap);
  return code;
}

#define GF_HIP_CHECK(expr)                                                                   \
  do {                                                                                       \
    hipError_t e_ = (expr);                                                                  \
    if (e_ != hipSuccess)                                                                    \
      return set_err(GF_E_HIP, "%s failed: %s", #expr, hipGetErrorString(e_));               \
  } while (0)

#define GF_LAUNCH_CHECK(name)                                                                \
  do {                                                                                       \
    hipError_t e_ = hipGetLastError();                                                       \
    if (e_ != hipSuccess)                                                                    \
      return set_err(GF_E_HIP, "launch of %s failed: %s", name, hipGetErrorString(e_));      \
  } while (0)

// ------------------------------------------------------------------------------------------
// Problem description (passed by value as a kernel argument).  Sizes are < 2^31 (checked).
struct Problem {
  int64_t K;
  int32_t M, N;
  int32_t tile_out, tile_in;
  int32_t R, C;  // tile rows / cols
  float sigma;
  float q_lo, q_hi;  // clamp range of the scaled quadratic form q * kHalfLog2e
  int32_t normalize;
  int32_t W;  // words per tile-row / tile-column mask (0: the ids are emitted by k_emit)
  int32_t S;  // backward accumulator stripes (power of two): tile t adds into stripe t % S
  int32_t mu_tanh;  // batched layers: mu holds mu_raw, the kernels use tanh(mu_raw) and d_mu
                    // receives dL/d(mu_raw) (GaussianLinear.materialize_mu)
  int32_t mask_clamp;  // clamp_quad < 80: the backward drops clamped pixels from the quadratic-
                       // form moments (at 80 and above their terms are below e^-40)
  int32_t heavy;  // > 0 (single fields on the k_bin_tiles path): tiles of more than `heavy`
                  // Gaussians are listed by k_bin_tiles and rendered / reduced by four waves
  // Capacity mode (gf_forward_kcap, gf_backward_direct_kcap): K above is the capacity, which
  // fixes the workspace layouts, mask words and launch grids; the live number of Gaussians is
  // *kdev and the live pair count *pdev, read by the kernels.  NULL: K and the host's pair count.
  const int64_t* kdev;
  const int64_t* pdev;
};

// The Gaussians the kernels take: K, or in capacity mode the device value clamped to [0, K].
__device__ inline int64_t live_k(const Problem& p) {
  if (!p.kdev) return p.K;
  const int64_t k = *p.kdev;
  return k < 0 ? 0 : (k > p.K ? p.K : k);
}

// The pair count the backward's saved-state checks use: num_pairs, or in capacity mode the
// forward's device value.
__device__ inline int64_t live_pairs(const Problem& p, int64_t num_pairs) { return p.pdev ? *p.pdev : num_pairs; }

// A Gaussian's mean coordinate i (0: row, 1: column) as the field uses it.
__device__ inline float mu_at(const Problem& p, const float* __restrict__ mu, int64_t i) {
  const float v = mu[i];
  return p.mu_tanh ? tanhf(v) : v;
}

// Per-Gaussian constants of the tile kernels: with dx = x - mu0, dy = y - mu1,
//   a = wa dx,  z = wb dx + wc dy,  q' = kHalfLog2e * (d^T cov^-1 d),
//   basis = 2^clamp(q') = exp(-q/2) with q clamped to [0, clamp]:
//   gen == 0 (positive-definite fp32 covariance): q' = -(a^2 + z^2);
//   gen != 0 (the fp32 covariance lost positive definiteness in rounding, det < 0):
//     q' = z^2 - a^2, the exact inverse of that indefinite matrix; its negative forms the clamp
//     maps to q = 0 (basis 1), as the reference's torch path does.
struct __align__(16) GaussEval {
  float mu0, mu1, wa, wb, wc, w;  // w = amp * norm
  int32_t gid;                    // the Gaussian's id (pair-ordered copies carry it)
  float gen;                      // 0: whitened form, 1: general form
};

struct WsHeader {
  uint32_t status;
  uint32_t heavy;      // forward, heavy-tile mode: tiles in the heavy-tile list
  int64_t* num_pairs;  // forward, tiles binned in the render: where the render stores P
  int64_t pairs;       // forward: P as the binning computed it, beside the status word, so that
                       // one 32-byte copy reads both back (gf_forward_bin's num_pairs_host)
  int64_t max_span;    // forward: the most tiles one Gaussian's rectangle covers (gf_bin_info)
  // forward, tiles binned in the render: per k_prep workgroup, the pairs of its Gaussians and
  // its widest rectangle, which the host read-back after the binning sums (gf_forward_bin's
  // num_pairs_host, gf_forward_bin_info) in the same copy as the status word
  int32_t part[16][2];
  uint32_t pad[24];
};
static_assert(sizeof(WsHeader) == 256, "workspace header must be 256 bytes");

size_t align256(size_t x) { return (x + 255) & ~size_t(255); }

// Forward workspace: header, per-Gaussian evaluation constants eval[K] (GaussEval), rect[K]
// (int4 tile ranges), cov[K] (float4: the fp32 covariance s00, s01, s11 and 0), fill[T]
// (int32 ids emitted so far into each tile's segment; emission path), rowmask[R][W] and
// colmask[C][W] (mask path: bit g%32 of word g/32 is set when Gaussian g's tile rectangle covers
// the tile row / column), bsq[blocks] (fp32 sum of delta-W^2 over each 16x16 block, written by
// the batched render for the layer's norm), dcoef[K][6] (float4, mask path: the chain-rule map
// of each Gaussian, see store_dcoef) and dgrad[K][8] (the gradients of gf_backward_direct, which
// the binning clears).
struct FwdLayout {
  size_t eval, rect, cov, lfac, fill, rowmask, colmask, bsq, dcoef, dgrad, total;
};
FwdLayout fwd_layout(const Problem& p) {
  const int64_t K = p.K, T = (int64_t)p.R * p.C;
  FwdLayout L;
  size_t o = sizeof(WsHeader);
  L.eval = o;
  o = align256(o + 32 * (size_t)K);
  L.rect = o;
  o = align256(o + sizeof(int4) * (size_t)K);
  L.cov = o;
  o = align256(o + sizeof(float4) * (size_t)K);
  L.lfac = o;  // (l11, l22) of each Gaussian's Cholesky factor, for the backward's finish
  o = align256(o + sizeof(float2) * (size_t)K);
  L.fill = o;  // emission path: per-tile fill counts; mask path: the heavy-tile list
  o = align256(o + sizeof(int32_t) * (size_t)T);
  L.rowmask = o;
  o = align256(o + sizeof(uint32_t) * (size_t)p.R * (size_t)p.W);
  L.colmask = o;
  o = align256(o + sizeof(uint32_t) * (size_t)p.C * (size_t)p.W);
  L.bsq = o;  // batched render: sum of squares of delta-W over each 16x16 block (block index sidx)
  o = align256(o + sizeof(float) * (size_t)T * (p.tile_out == 32 && p.tile_in == 32 ? 4 : 1));
  L.dcoef = o;  // the binning (k_bin_tiles or k_prep): each Gaussian's chain-rule map (six float4)
  o = align256(o + 6 * sizeof(float4) * (size_t)K);
  L.dgrad = o;  // gf_backward_direct's gradients: [K][8] (d_amp, d_mu x2, d_chol_raw x3, 2 unused)
  o = align256(o + 8 * sizeof(float) * (size_t)K);
  L.total = o;
  return L;
}

// Backward workspace: header + S stripes of eight fp32 accumulators per Gaussian, stripe-major
// (acc[s][g][8], see acc_slot): the tiles of a Gaussian spread their atomics over S addresses
// per moment, on S different cache lines.
// It must be zero before the first backward; every backward leaves it zero again
// (k_bwd_finish clears what it reads), so a workspace kept across calls is zeroed once.
struct BwdLayout {
  size_t acc, total;
};
BwdLayout bwd_layout(const Problem& p) {
  BwdLayout L;
  size_t o = sizeof(WsHeader);
  L.acc = o;
  o = align256(o + sizeof(float) * 8 * (size_t)p.S * (size_t)p.K);
  L.total = o;
  return L;
}

__device__ inline void set_status(uint32_t* status, uint32_t bit) { atomicOr(status, bit); }

// Accumulator slot (eight floats) of stripe st of Gaussian g.  Stripe-major: atomics on one
// cache line serialise where they are performed, so a Gaussian that touches thousands of
// tiles must not keep its S stripes on one or two lines (Gaussian-major, 128-byte lines hold
// four 32-byte slots).
__device__ inline int64_t acc_slot(const Problem& p, int64_t g, int64_t st) { return st * p.K + g; }

// Index in dgrad of gradient k of Gaussian g, k in the order of the chain-rule map: d_amp, d_mu
// (2), d_chol_raw (3).  One 32-byte slot per Gaussian: its six atomics stay on one cache line,
// which four Gaussians share (as the moment accumulators); three arrays of 4, 8 and 12 bytes
// per Gaussian put up to 32 Gaussians on a line, and the atomics serialised on them (cfg3's
// backward: 15.8 us against 9.2 us).
__device__ inline uint32_t direct_slot(int32_t g, int k) { return 8 * (uint32_t)g + (uint32_t)k; }

__device__ inline int32_t clamp_i32(int32_t v, int32_t lo, int32_t hi) {
  return v < lo ? lo : (v > hi ? hi : v);
}

// Bit-exact tile rectangle of a Gaussian from its fp32 covariance (same fp32 operation
// sequence as gf_tile_rect, with the row/column indices, already clamped into [0, M-1],
// divided in 32-bit integers).
__device__ inline int4 bin_rect(const Problem& p, float mu0, float mu1, GfCov c, int32_t* touched) {
#pragma clang fp contract(off)
  const float std_r = gf_sqrt_rn(gf_clamp_min_nan(c.s00, GF_COV_FLOOR));
  const float std_c = gf_sqrt_rn(gf_clamp_min_nan(c.s11, GF_COV_FLOOR));
  const float centre_r = ((mu0 + 1.0f) * 0.5f) * (float)(p.M - 1);
  const float centre_c = ((mu1 + 1.0f) * 0.5f) * (float)(p.N - 1);
  const float half_r = ((p.sigma * std_r) * 0.5f) * (float)(p.M - 1 > 1 ? p.M - 1 : 1);
  const float half_c = ((p.sigma * std_c) * 0.5f) * (float)(p.N - 1 > 1 ? p.N - 1 : 1);
  const int32_t row_lo = (int32_t)gf_clamp_i64(gf_f32_to_i64_torch(__builtin_floorf(centre_r - half_r)), 0, p.M - 1);
  const int32_t row_hi = (int32_t)gf_clamp_i64(gf_f32_to_i64_torch(__builtin_ceilf(centre_r + half_r)), 0, p.M - 1);
  const int32_t col_lo = (int32_t)gf_clamp_i64(gf_f32_to_i64_torch(__builtin_floorf(centre_c - half_c)), 0, p.N - 1);
  const int32_t col_hi = (int32_t)gf_clamp_i64(gf_f32_to_i64_torch(__builtin_ceilf(centre_c + half_c)), 0, p.N - 1);
  int4 r;
  r.x = clamp_i32(row_lo / p.tile_out, 0, p.R - 1);
  r.y = clamp_i32(row_hi / p.tile_out, 0, p.R - 1);
  r.z = clamp_i32(col_lo / p.tile_in, 0, p.C - 1);
  r.w = clamp_i32(col_hi / p.tile_in, 0, p.C - 1);
  *touched = (r.y - r.x + 1) * (r.w - r.z + 1);
  return r;
}

// Evaluation constants of a Gaussian: the Cholesky factor L' of its fp32 covariance and
// R = L'^-1 in double (R^T R = cov^-1), scaled by sqrt(log2(e)/2) and rounded once.
__device__ inline GaussEval eval_from_cov(const Problem& p, float mu0, float mu1, GfCov c, float amp) {
  const double a = (double)c.s00, b = (double)c.s01, d = (double)c.s11;
  const double det_signed = a * d - b * b;  // exact products, one rounding
  double det = det_signed;
  GaussEval v;
  v.mu0 = mu0;
  v.mu1 = mu1;
  // d^T cov^-1 d = dx^2 / a + (a / det) (dy - (b / a) dx)^2 for any det != 0 (a > 0): the
  // second coefficient takes the sign of det, so an indefinite matrix only flips that term.
  v.gen = det < 0.0 ? 1.0f : 0.0f;
  det = fabs(det);
  if (!(det > 0.0)) det = 1e-300;  // exactly singular fp32 covariance: a degenerate line
  const double r00 = 1.0 / sqrt(a);
  const double r11 = sqrt(a / det);  // 1 / l22 with l22 = sqrt(det / a)
  const double r10 = -(b / a) * r11;  // -l21 / (l11 l22)
  v.wa = (float)(kSqrtHalfLog2e * r00);
  v.wb = (float)(kSqrtHalfLog2e * r10);
  v.wc = (float)(kSqrtHalfLog2e * r11);
  float norm = 1.0f;
  if (p.normalize) {
#pragma clang fp contract(off)
    // 1 / (2 pi max(sqrt(det), eps)) on the signed det: an indefinite covariance gives NaN, as
    // torch.clamp keeps the NaN of sqrt(det < 0) in the reference (gaussian_core.py:55-82)
    const float sq = gf_sqrt_rn((float)det_signed);
    norm = gf_div_f32(1.0f, GF_TWO_PI_F32 * (sq < GF_FLT_EPS ? GF_FLT_EPS : sq));
  }
  v.w = amp * norm;
  v.gid = -1;
  return v;
}

__device__ inline GaussEval eval_geom(const Problem& p, const float* __restrict__ mu,
                                      const float* __restrict__ chol_raw,
                                      const float* __restrict__ amp, int64_t g) {
  const GfChol L = gf_activate_cholesky(chol_raw[3 * g + 0], chol_raw[3 * g + 1], chol_raw[3 * g + 2]);
  return eval_from_cov(p, mu_at(p, mu, 2 * g + 0), mu_at(p, mu, 2 * g + 1), gf_cov_from_chol(L),
                       amp ? amp[g] : 0.0f);
}

__device__ inline GaussEval load_eval(const GaussEval* __restrict__ ev, int64_t g) {
  const float4* q = reinterpret_cast<const float4*>(ev + g);
  const float4 a = q[0], b = q[1];
  GaussEval v;
  v.mu0 = a.x;
  v.mu1 = a.y;
  v.wa = a.z;
  v.wb = a.w;
  v.wc = b.x;
  v.w = b.y;
  v.gid = __float_as_int(b.z);
  v.gen = b.w;
  return v;
}

__device__ inline GaussEval zero_eval() {
  GaussEval v;
  v.mu0 = v.mu1 = v.wa = v.wb = v.wc = v.w = v.gen = 0.0f;
  v.gid = -1;
  return v;
}

// 2^clamp(q'), q' = -(A + z^2).
__device__ inline float basis_w(const Problem& p, float A, float z) {
  // q' <= 0 for the definite form, so the upper clamp (p.q_hi: 0, or +inf without a clamp)
  // is the literal 0: an inline constant, which leaves med3 its one scalar operand for q_lo.
  const float q = -fmaf(z, z, A);
  return __builtin_amdgcn_exp2f(__builtin_amdgcn_fmed3f(q, p.q_lo, 0.0f));
}

// q' of a pixel for either form of GaussEval.
__device__ inline float quad_form(const GaussEval& u, float dx, float dy) {
  const float a = u.wa * dx;
  const float z = fmaf(u.wc, dy, u.wb * dx);
  return u.gen != 0.0f ? fmaf(z, z, -(a * a)) : -fmaf(z, z, a * a);
}

__device__ inline float basis_q(const Problem& p, float q) {
  return __builtin_amdgcn_exp2f(__builtin_amdgcn_fmed3f(q, p.q_lo, p.q_hi));
}

__device__ inline float readlane_f(float v, int lane) {
  return __int_as_float(__builtin_amdgcn_readlane(__float_as_int(v), lane));
}

__device__ inline int64_t readlane_i64(int64_t v, int lane) {
  const uint32_t lo = (uint32_t)__builtin_amdgcn_readlane((int32_t)(uint32_t)v, lane);
  const uint32_t hi = (uint32_t)__builtin_amdgcn_readlane((int32_t)(v >> 32), lane);
  return (int64_t)(((uint64_t)hi << 32) | lo);
}

// Orders the memory operations of one wave whose lanes exchange data through LDS: release /
// acquire fences at wavefront scope (the LDS performs one wave's operations in issue order, so
// they cost no wait instruction; rocPRIM's wave_barrier is the same) and a wave barrier that
// keeps the compiler from moving code across.
__device__ inline void wave_sync() {
  __builtin_amdgcn_fence(__ATOMIC_RELEASE, "wavefront");
  __builtin_amdgcn_wave_barrier();
  __builtin_amdgcn_fence(__ATOMIC_ACQUIRE, "wavefront");
}

// The same where lanes exchange data through global memory (rare paths): a workgroup-scope
// fence, which waits for the wave's outstanding memory operations.
__device__ inline void wave_sync_global() {
  __builtin_amdgcn_fence(__ATOMIC_SEQ_CST, "workgroup");
  __builtin_amdgcn_wave_barrier();
}

// Streaming access to delta-W (written once by the render) and dL/d(delta-W) (read once by the
// backward): the nontemporal hint keeps those bytes from evicting the L2 lines the tile kernels
// reuse (masks, Gaussian constants, coordinates, accumulators).
typedef float f32x4_t __attribute__((ext_vector_type(4)));
__device__ inline void store4_stream(float* q, float a, float b, float c, float d) {
  const f32x4_t v = {a, b, c, d};
  __builtin_nontemporal_store(v, reinterpret_cast<f32x4_t*>(q));
}
__device__ inline void store_stream(float* q, float v) { __builtin_nontemporal_store(v, q); }
__device__ inline float4 load4_stream(const float* q) {
  const f32x4_t v = __builtin_nontemporal_load(reinterpret_cast<const f32x4_t*>(q));
  return make_float4(v.x, v.y, v.z, v.w);
}
__device__ inline float load_stream(const float* q) { return __builtin_nontemporal_load(q); }

// The merged consumer of a batched layer (gf_layer.merged_weight): besides (or instead of) delta-W
// the render writes merged = base + scale * delta-W, each element rounded as the fp32 multiply and
// then the fp32 add of `weight + delta_weight * adapter_scale` (GaussianLinear, delta_apply
// "merged"), with no contraction into an FMA.
struct MergedOut {
  const float* base;  // [M*N], the frozen base weight
  float* merged;      // [M*N] out; NULL: no merged output
  float scale;
};

__device__ inline float merge_weight(float w, float scale, float d) {
#pragma clang fp contract(off)
  const float prod = d * scale;  // two roundings, as torch's two elementwise kernels
  return w + prod;
}

// Columns pc .. pc+3 of row pr (those inside the matrix) of delta-W from v[], and of the merged
// weight where there is one.  delta may be NULL (a merged layer whose delta-W is not kept).
__device__ inline void store_row4(const Problem& p, float* __restrict__ delta, const MergedOut& mo, int32_t pr,
                                  int32_t pc, const float (&v)[4], bool tile_inner = false) {
  const int64_t off = (int64_t)pr * p.N + pc;
  const bool inner = pc + 3 < p.N;
  // tile_inner (the same in every lane): the lane's tile lies inside the matrix, so with rows of
  // N % 4 == 0 floats from a 16-byte aligned base every lane's float4 is inside and aligned --
  // a scalar test instead of per-lane ones
  const bool rows4 = tile_inner && (p.N & 3) == 0;
  if (delta) {
    float* out = delta + off;
    if ((rows4 && (reinterpret_cast<uintptr_t>(delta) & 15) == 0) ||
        (inner && (reinterpret_cast<uintptr_t>(out) & 15) == 0)) {
      store4_stream(out, v[0], v[1], v[2], v[3]);
    } else {
#pragma unroll
      for (int i = 0; i < 4; ++i)
        if (pc + i < p.N) store_stream(out + i, v[i]);
    }
  }
  if (mo.merged) {
    const float* w = mo.base + off;
    float* out = mo.merged + off;
    if ((rows4 && ((reinterpret_cast<uintptr_t>(mo.merged) | reinterpret_cast<uintptr_t>(mo.base)) & 15) == 0) ||
        (inner && ((reinterpret_cast<uintptr_t>(out) | reinterpret_cast<uintptr_t>(w)) & 15) == 0)) {
      const float4 w4 = load4_stream(w);
      store4_stream(out, merge_weight(w4.x, mo.scale, v[0]), merge_weight(w4.y, mo.scale, v[1]),
                    merge_weight(w4.z, mo.scale, v[2]), merge_weight(w4.w, mo.scale, v[3]));
    } else {
#pragma unroll
      for (int i = 0; i < 4; ++i)
        if (pc + i < p.N) store_stream(out + i, merge_weight(load_stream(w + i), mo.scale, v[i]));
    }
  }
}


// ------------------------------------------------------------------------------------------
// DPP wave primitives (gfx9 row_shr / row_bcast; no LDS traffic).

template <int CTRL, int ROWS>
__device__ inline int32_t dpp_i32(int32_t v) {
  return __builtin_amdgcn_update_dpp(0, v, CTRL, ROWS, 0xf, false);
}

// Inclusive scan over the 64 lanes: row_shr 1,2,4,8 within rows of 16, then row_bcast 15 / 31.
__device__ inline int32_t dpp_scan_i32(int32_t v) {
  v += dpp_i32<0x111, 0xf>(v);
  v += dpp_i32<0x112, 0xf>(v);
  v += dpp_i32<0x114, 0xf>(v);
  v += dpp_i32<0x118, 0xf>(v);
  v += dpp_i32<0x142, 0xa>(v);
  v += dpp_i32<0x143, 0xc>(v);
  return v;
}

template <int CTRL, int ROWS>
__device__ inline int64_t dpp_i64(int64_t v) {
  const int32_t lo = __builtin_amdgcn_update_dpp(0, (int32_t)(uint32_t)v, CTRL, ROWS, 0xf, false);
  const int32_t hi = __builtin_amdgcn_update_dpp(0, (int32_t)(v >> 32), CTRL, ROWS, 0xf, false);
  return (int64_t)(((uint64_t)(uint32_t)hi << 32) | (uint32_t)lo);
}

__device__ inline int64_t dpp_scan_i64(int64_t v) {
  v += dpp_i64<0x111, 0xf>(v);
  v += dpp_i64<0x112, 0xf>(v);
  v += dpp_i64<0x114, 0xf>(v);
  v += dpp_i64<0x118, 0xf>(v);
  v += dpp_i64<0x142, 0xa>(v);
  v += dpp_i64<0x143, 0xc>(v);
  return v;
}

template <int CTRL>
__device__ inline float dpp_f32(float v) {
  return __int_as_float(dpp_i32<CTRL, 0xf>(__float_as_int(v)));
}

// Inclusive scan over the 64 lanes in fp32 (the order of dpp_scan_i32): lane 63 holds the
// wave's sum, in a fixed order.
__device__ inline float dpp_scan_f32(float v) {
  v += __int_as_float(dpp_i32<0x111, 0xf>(__float_as_int(v)));
  v += __int_as_float(dpp_i32<0x112, 0xf>(__float_as_int(v)));
  v += __int_as_float(dpp_i32<0x114, 0xf>(__float_as_int(v)));
  v += __int_as_float(dpp_i32<0x118, 0xf>(__float_as_int(v)));
  v += __int_as_float(dpp_i32<0x142, 0xa>(__float_as_int(v)));
  v += __int_as_float(dpp_i32<0x143, 0xc>(__float_as_int(v)));
  return v;
}

// Sum over each row of 16 lanes, left in lane 15 of the row (other lanes hold partial sums).
__device__ inline float dpp_row_sum_f32(float v) {
  v += __int_as_float(dpp_i32<0x111, 0xf>(__float_as_int(v)));
  v += __int_as_float(dpp_i32<0x112, 0xf>(__float_as_int(v)));
  v += __int_as_float(dpp_i32<0x114, 0xf>(__float_as_int(v)));
  v += __int_as_float(dpp_i32<0x118, 0xf>(__float_as_int(v)));
  return v;
}

// Sum over each row of 16 lanes, in every lane of the row: xor butterflies (quad_perm [1,0,3,2],
// [2,3,0,1], row_half_mirror, row_mirror), each lane adding the same two halves.
__device__ inline float dpp_row_allsum_f32(float v) {
  v += dpp_f32<0xb1>(v);
  v += dpp_f32<0x4e>(v);
  v += dpp_f32<0x141>(v);
  v += dpp_f32<0x140>(v);
  return v;
}

// dst = src[partner] + src in the lanes 8..15 of each row of 16 (DPP banks 2 and 3), partner
// = 15 - lane (row_mirror); dst unchanged in lanes 0..7 (the bank mask leaves them unwritten).
// One v_add_f32_dpp where a select per operand would take three instructions; the s_nop gives
// the two wait states a DPP read needs after a VALU write of its source.
__device__ inline float row_mirror_sum_upper(float dst, float src) {
  __asm__("s_nop 1\n\tv_add_f32_dpp %0, %1, %1 row_mirror row_mask:0xf bank_mask:0xc" : "+v"(dst) : "v"(src));
  return dst;
}

// The same in lanes 4..7 and 12..15 of each row (banks 1 and 3), partner = lane ^ 7 within
// each half row (row_half_mirror).
__device__ inline float row_half_mirror_sum_odd_banks(float dst, float src) {
  __asm__("s_nop 1\n\tv_add_f32_dpp %0, %1, %1 row_half_mirror row_mask:0xf bank_mask:0xa" : "+v"(dst) : "v"(src));
  return dst;
}

// v + v[lane ^ 1] in every lane, as one DPP add where the wave's lanes all still run (volatile:
// not moved into a branch whose lanes are a subset, where the partner's value would not be read).
__device__ inline float pair_sum_all_lanes(float v) {
  float r;
  __asm__ volatile("s_nop 1\n\tv_add_f32_dpp %0, %1, %1 quad_perm:[1,0,3,2] row_mask:0xf bank_mask:0xf" : "=v"(r) : "v"(v));
  return r;
}

// ------------------------------------------------------------------------------------------
// Workgroup scans.

__device__ inline int64_t wave_inclusive_scan(int64_t x) { return dpp_scan_i64(x); }

// Exclusive scan across a workgroup of BLOCK threads; *total receives the sum.
// lds must hold BLOCK/64 + 1 int64.
template <int BLOCK>
__device__ int64_t block_exclusive_scan(int64_t v, int64_t* total, int64_t* lds) {
  constexpr int kWaves = BLOCK / 64;
  const int lane = threadIdx.x & 63, wid = threadIdx.x >> 6;
  const int64_t inc = wave_inclusive_scan(v);
  if (lane == 63) lds[wid] = inc;
  __syncthreads();
  if (wid == 0) {
    const int64_t w = lane < kWaves ? lds[lane] : 0;
    const int64_t wi = wave_inclusive_scan(w);
    if (lane < kWaves) lds[lane] = wi - w;
    if (lane == kWaves - 1) lds[kWaves] = wi;
  }
  __syncthreads();
  const int64_t excl = inc - v + lds[wid];
  *total = lds[kWaves];
  __syncthreads();
  return excl;
}

// In-place exclusive scan of data[0..n) by one workgroup; returns the total.  Each thread
// owns a contiguous run of ceil(n/BLOCK) elements.
template <int BLOCK>
__device__ int64_t block_scan_runs(int64_t* data, int64_t n, int64_t* lds) {
  const int64_t per = (n + BLOCK - 1) / BLOCK;
  const int64_t b = (int64_t)threadIdx.x * per;
  const int64_t e = b + per < n ? b + per : n;
  int64_t s = 0;
  for (int64_t i = b; i < e; ++i) s += data[i];
  int64_t total;
  int64_t run = block_exclusive_scan<BLOCK>(s, &total, lds);
  for (int64_t i = b; i < e; ++i) {
    const int64_t v = data[i];
    data[i] = run;
    run += v;
  }
  __syncthreads();
  return total;
}

// ------------------------------------------------------------------------------------------
// k_bin: one workgroup.

__device__ inline void store_eval(GaussEval* ev, int64_t i, const GaussEval& v) {
  float4* q = reinterpret_cast<float4*>(ev + i);
  q[0] = make_float4(v.mu0, v.mu1, v.wa, v.wb);
  q[1] = make_float4(v.wc, v.w, __int_as_float(v.gid), v.gen);
}

__device__ inline GaussEval readlane_eval(const GaussEval& v, int lane) {
  GaussEval r;
  r.mu0 = readlane_f(v.mu0, lane);
  r.mu1 = readlane_f(v.mu1, lane);
  r.wa = readlane_f(v.wa, lane);
  r.wb = readlane_f(v.wb, lane);
  r.wc = readlane_f(v.wc, lane);
  r.w = readlane_f(v.w, lane);
  r.gid = __builtin_amdgcn_readlane(v.gid, lane);
  r.gen = readlane_f(v.gen, lane);
  return r;
}

// Gaussians g = threadIdx.x + i * kBinThreads, i < kBinRectRegs, keep their tile rectangle in
// registers between the phases of k_bin; the rest re-read it from the workspace.
constexpr int kBinRectRegs = 4;

// One wave scans whole rows of the band's difference array (lane l holds columns
// j0 + l*V .. +V-1): counts are the inclusive prefix of the differences along the row, and
// tile_ptr of a tile is its row's base plus the exclusive prefix of the counts.  Writes
// tile_ptr and clears the tiles' fill counters directly.
template <int V>
__device__ inline void bin_scan_rows(const int32_t* lds, int32_t stride, int32_t C, int32_t nb, int64_t b0,
                                     const int64_t* rowbase, int64_t* __restrict__ tile_ptr,
                                     int32_t* __restrict__ fill, int lane, int wid) {
  // fill == nullptr: no emission follows (mask path), nothing to clear
  for (int32_t row = wid; row < nb; row += kBinThreads / 64) {
    const int32_t* rp = lds + row * stride;
    const int64_t out0 = (b0 + row) * (int64_t)C;
    const int64_t base_off = rowbase[row];
    int32_t carry_d = 0, carry_c = 0;
    for (int32_t j0 = 0; j0 < C; j0 += 64 * V) {
      const int32_t col0 = j0 + lane * V;
      int32_t c[V];
      int32_t run = 0;
#pragma unroll
      for (int v = 0; v < V; ++v) {
        run += (col0 + v < C) ? rp[col0 + v] : 0;
        c[v] = run;
      }
      const int32_t dinc = dpp_scan_i32(run);
      const int32_t before = carry_d + dinc - run;  // count carried into this lane's first column
      int32_t csum = 0;
#pragma unroll
      for (int v = 0; v < V; ++v) {
        c[v] = (col0 + v < C) ? c[v] + before : 0;
        csum += c[v];
      }
      const int32_t cinc = dpp_scan_i32(csum);
      int32_t off = carry_c + cinc - csum;
#pragma unroll
      for (int v = 0; v < V; ++v) {
        if (col0 + v < C) {
          tile_ptr[out0 + col0 + v] = base_off + off;
          if (fill) fill[out0 + col0 + v] = 0;
        }
        off += c[v];
      }
      carry_d += __builtin_amdgcn_readlane(dinc, 63);
      carry_c += __builtin_amdgcn_readlane(cinc, 63);
    }
  }
}

// The binning of one field by one workgroup of kBinThreads threads.  With kEval it also
// stores each Gaussian's evaluation constants (one Gaussian per thread); otherwise k_emit
// computes them.  With p.W > 0 (mlds: kMaskLdsWords of LDS) it also writes the tile-row and
// tile-column masks, from which the render reads each tile's ids (no emission).
template <bool kEval>
__device__ __forceinline__ void bin_body(const Problem& p, const float* __restrict__ mu,
                                         const float* __restrict__ chol_raw,
                                         const float* __restrict__ amp,
                                         int64_t* __restrict__ tile_ptr,
                                         int64_t* __restrict__ num_pairs, uint8_t* ws,
                                         const FwdLayout& L, uint32_t* mlds) {
  __shared__ int32_t lds[kLdsDiffWords];
  __shared__ int64_t rowbase[kBinMaxBandRows + 1];
  __shared__ int32_t rowdiff[kBinMaxBandRows + 1];
  __shared__ int64_t scan_lds[kBinThreads / 64 + 1];
  __shared__ unsigned long long pairs_lds;
  __shared__ int32_t span_lds;  // the most tiles of one rectangle
  // rectangles with long row / column spans: Gaussian, first row / column in the band, span,
  // columns (row spans), and the prefix of the spans
  __shared__ int32_t long_g[kLongMax], long_lo[kLongMax], long_n[kLongMax];
  __shared__ int32_t long_c0[kLongMax], long_c1[kLongMax], long_off[kLongMax + 1];
  __shared__ uint32_t nlong;
  WsHeader* hdr = reinterpret_cast<WsHeader*>(ws);
  int4* rect = reinterpret_cast<int4*>(ws + L.rect);
  float4* covs = reinterpret_cast<float4*>(ws + L.cov);
  int32_t* fill = reinterpret_cast<int32_t*>(ws + L.fill);
  uint32_t* rowmask = reinterpret_cast<uint32_t*>(ws + L.rowmask);
  uint32_t* colmask = reinterpret_cast<uint32_t*>(ws + L.colmask);
  const int64_t K = p.K, T = (int64_t)p.R * p.C;
  const int lane = threadIdx.x & 63, wid = threadIdx.x >> 6;
  const int32_t W = mlds ? p.W : 0;  // mask words (the host only sets p.W where masks fit)
  if (threadIdx.x == 0) {
    hdr->status = 0u;
    pairs_lds = 0ull;
    span_lds = 0;
    nlong = 0u;
  }

  // Per-tile counts go through LDS, band by band of whole tile rows, when the grid allows it.
  const bool lds_path = bin_counts_in_lds(p.C, K);
  const int32_t C = p.C;
  // LDS rows of masks are Wp = W | 1 words apart: with an odd stride, the same word of
  // different rows falls in different LDS banks (the lanes of a wave share a word index).
  const int32_t Wp = W > 0 ? (W | 1) : 0;  // no masks: no mask rows (mlds may be NULL)
  // Count rows likewise Cp = C | 1 apart (the first columns of clustered rectangles coincide).
  const int32_t Cp = C | 1;
  int32_t band_rows = lds_path ? min(kLdsDiffWords / Cp, kBinMaxBandRows) : 0;
  if (W > 0) band_rows = min(band_rows, kMaskLdsWords / Wp);
  auto clear_band = [&](int32_t nb) {
    for (int32_t i = threadIdx.x; i < nb * Cp; i += kBinThreads) lds[i] = 0;
    for (int32_t i = threadIdx.x; i <= nb; i += kBinThreads) rowdiff[i] = 0;
    for (int32_t i = threadIdx.x; i < nb * Wp; i += kBinThreads) mlds[i] = 0u;
  };
  // n mask rows of LDS (stride Wp) -> global rows of W words, by threads t0, t0 + nt, ...
  auto copy_masks = [&](uint32_t* out, int32_t n, int32_t t0, int32_t nt) {
    for (int32_t i = t0; i < n * W; i += nt) {
      const int32_t r = i / W;
      out[i] = mlds[r * Wp + (i - r * W)];
    }
  };
  if (lds_path) clear_band(min(band_rows, p.R));
  // The nl listed long spans, item by item (entry e covers long_n[e] rows / columns from
  // long_lo[e]): wave 0 scans the spans, then thread t takes a contiguous run of the items.
  // Every thread must call it (barriers); it ends with a barrier.
  auto run_long = [&](int32_t nl, auto&& item) {
    if (wid == 0) {
      int32_t carry = 0;
      for (int32_t e0 = 0; e0 < nl; e0 += 64) {
        const int32_t e = e0 + lane;
        const int32_t v = e < nl ? long_n[e] : 0;
        const int32_t inc = dpp_scan_i32(v);
        if (e < nl) long_off[e] = carry + inc - v;
        carry += __builtin_amdgcn_readlane(inc, 63);
      }
      if (lane == 0) long_off[nl] = carry;
    }
    __syncthreads();
    const int32_t total = long_off[nl];
    const int32_t per = (total + kBinThreads - 1) / kBinThreads;
    int32_t i = (int32_t)threadIdx.x * per;
    const int32_t iend = min(i + per, total);
    if (i < iend) {
      int32_t lo = 0, hi = nl;  // long_off[lo] <= i < long_off[hi]
      while (hi - lo > 1) {
        const int32_t mid = (lo + hi) >> 1;
        if (long_off[mid] <= i) lo = mid;
        else hi = mid;
      }
      int32_t e = lo, k = i - long_off[lo];
      for (; i < iend; ++i, ++k) {
        while (k >= long_n[e]) {  // spans are >= 1
          k -= long_n[e];
          ++e;
        }
        item(e, long_lo[e] + k);
      }
    }
    __syncthreads();
  };
  // Appends a long span to the list; false when the list is full (the caller loops itself).
  auto push_long = [&](int64_t g, int32_t lo, int32_t n, int32_t c0, int32_t c1) -> bool {
    const uint32_t slot = atomicAdd(&nlong, 1u);
    if (slot >= (uint32_t)kLongMax) return false;
    long_g[slot] = (int32_t)g;
    long_lo[slot] = lo;
    long_n[slot] = n;
    long_c0[slot] = c0;
    long_c1[slot] = c1;
    return true;
  };

  // A: tile rectangles, fp32 covariances and pairs (tiles touched); the first
  // kBinRectRegs * kBinThreads Gaussians keep their rectangle in registers.
  int4 myrect[kBinRectRegs];
  int64_t my_pairs = 0;
  int32_t my_span = 0;
  struct PrepIn {
    float mu0, mu1, r11, r21, r22, amp;
  };
  auto load_in = [&](int64_t g) -> PrepIn {
    return PrepIn{mu_at(p, mu, 2 * g + 0), mu_at(p, mu, 2 * g + 1), chol_raw[3 * g + 0], chol_raw[3 * g + 1],
                  chol_raw[3 * g + 2], kEval ? amp[g] : 0.0f};
  };
  auto prep = [&](int64_t g, const PrepIn& in) -> int4 {
    const GfChol Lc = gf_activate_cholesky(in.r11, in.r21, in.r22);
    const GfCov c = gf_cov_from_chol(Lc);
    int32_t touched;
    const int4 r = bin_rect(p, in.mu0, in.mu1, c, &touched);
    rect[g] = r;
    covs[g] = make_float4(c.s00, c.s01, c.s11, 0.0f);
    reinterpret_cast<float2*>(ws + L.lfac)[g] = make_float2(Lc.l11, Lc.l22);
    my_pairs += touched;
    my_span = max(my_span, touched);
    if (kEval) {
      GaussEval v = eval_from_cov(p, in.mu0, in.mu1, c, in.amp);
      v.gid = (int32_t)g;
      store_eval(reinterpret_cast<GaussEval*>(ws + L.eval), g, v);
    }
    return r;
  };
#pragma unroll
  for (int i = 0; i < kBinRectRegs; ++i) {
    const int64_t g = threadIdx.x + (int64_t)i * kBinThreads;
    myrect[i] = make_int4(1, 0, 1, 0);  // empty
    if (g < K) myrect[i] = prep(g, load_in(g));
  }
  for (int64_t g = threadIdx.x + (int64_t)kBinRectRegs * kBinThreads; g < K; g += kBinThreads)
    prep(g, load_in(g));
  // B: P = total pairs: wave sums, one LDS atomic per wave after the barrier that orders them
  // behind the counter's initialisation; read by thread 0 after later barriers.
  const int64_t wave_pairs = readlane_i64(wave_inclusive_scan(my_pairs), 63);
  for (int off = 32; off > 0; off >>= 1) my_span = max(my_span, __shfl_xor(my_span, off));
  __syncthreads();
  if (lane == 0) {
    atomicAdd(&pairs_lds, (unsigned long long)wave_pairs);
    atomicMax(&span_lds, my_span);
  }

  // C: each covered row of each rectangle adds +1 at its first column and -1 after its last;
  // the rectangle's width is added over its rows through a difference array over rows (and,
  // with masks, the Gaussian's bit is set in each covered row's mask).  Wave 0 turns the row
  // differences into row totals and row bases while the other waves copy out the band's row
  // masks; then one wave per row scans the column differences into counts and the counts into
  // tile_ptr (row base + exclusive prefix), written coalesced together with cleared fill
  // counters (emission path).
  int64_t Pc = 0;
  if (lds_path) {
    int64_t band_base = 0;
    for (int32_t b0 = 0; b0 < p.R; b0 += band_rows) {
      const int32_t nb = min(p.R - b0, band_rows);
      if (b0 > 0) {
        clear_band(nb);
        __syncthreads();
      }
      auto row_item = [&](int32_t row, int32_t c0, int32_t c1, int64_t g) {
        int32_t* d = lds + (row - b0) * Cp;
        atomicAdd(d + c0, 1);
        if (c1 + 1 < C) atomicAdd(d + c1 + 1, -1);
        if (W > 0) atomicOr(mlds + (row - b0) * Wp + (int32_t)(g >> 5), 1u << (g & 31));
      };
      auto diff = [&](const int4 r, int64_t g) {
        const int32_t rlo = max(r.x, b0), rhi = min(r.y, b0 + nb - 1);
        if (rlo > rhi) return;
        const int32_t w = r.w - r.z + 1;
        atomicAdd(rowdiff + (rlo - b0), w);
        atomicAdd(rowdiff + (rhi + 1 - b0), -w);  // index <= nb
        if (rhi - rlo >= kLongSpan && push_long(g, rlo, rhi - rlo + 1, r.z, r.w)) return;
        for (int32_t row = rlo; row <= rhi; ++row) row_item(row, r.z, r.w, g);
      };
#pragma unroll
      for (int i = 0; i < kBinRectRegs; ++i) diff(myrect[i], threadIdx.x + (int64_t)i * kBinThreads);
      for (int64_t g = threadIdx.x + (int64_t)kBinRectRegs * kBinThreads; g < K; g += kBinThreads)
        diff(rect[g], g);
      __syncthreads();
      const int32_t nl = (int32_t)min(nlong, (uint32_t)kLongMax);
      if (nl > 0) {
        run_long(nl, [&](int32_t e, int32_t row) { row_item(row, long_c0[e], long_c1[e], long_g[e]); });
        if (threadIdx.x == 0) nlong = 0u;  // every thread read it before run_long's barriers
      }
      if (wid == 0) {
        int64_t carry = 0;
        int32_t carry_t = 0;
        for (int32_t r0 = 0; r0 < nb; r0 += 64) {
          const int32_t r = r0 + lane;
          const int32_t dv = r < nb ? rowdiff[r] : 0;
          const int32_t tinc = dpp_scan_i32(dv);
          const int64_t tot = r < nb ? (int64_t)(carry_t + tinc) : 0;  // row total
          const int64_t inc = wave_inclusive_scan(tot);
          if (r < nb) rowbase[r] = band_base + carry + inc - tot;
          carry += readlane_i64(inc, 63);
          carry_t += __builtin_amdgcn_readlane(tinc, 63);
        }
        if (lane == 0) rowbase[kBinMaxBandRows] = band_base + carry;
      } else if (W > 0) {
        copy_masks(rowmask + (int64_t)b0 * W, nb, threadIdx.x - 64, kBinThreads - 64);
      }
      __syncthreads();
      int32_t* fl = W > 0 ? nullptr : fill;
      if (C <= 64) bin_scan_rows<1>(lds, Cp, C, nb, b0, rowbase, tile_ptr, fl, lane, wid);
      else if (C <= 128) bin_scan_rows<2>(lds, Cp, C, nb, b0, rowbase, tile_ptr, fl, lane, wid);
      else bin_scan_rows<4>(lds, Cp, C, nb, b0, rowbase, tile_ptr, fl, lane, wid);
      band_base = rowbase[kBinMaxBandRows];
      __syncthreads();
    }
    Pc = band_base;
    // D (masks): the column masks, band by band of tile columns.
    if (W > 0) {
      const int32_t band_cols = kMaskLdsWords / Wp;
      for (int32_t cb0 = 0; cb0 < C; cb0 += band_cols) {
        const int32_t nc = min(C - cb0, band_cols);
        for (int32_t i = threadIdx.x; i < nc * Wp; i += kBinThreads) mlds[i] = 0u;
        __syncthreads();
        auto col_item = [&](int32_t c, int64_t g) {
          atomicOr(mlds + (c - cb0) * Wp + (int32_t)(g >> 5), 1u << (g & 31));
        };
        auto colset = [&](const int4 r, int64_t g) {
          const int32_t lo = max(r.z, cb0), hi = min(r.w, cb0 + nc - 1);
          if (lo > hi) return;
          if (hi - lo >= kLongSpan && push_long(g, lo, hi - lo + 1, 0, 0)) return;
          for (int32_t c = lo; c <= hi; ++c) col_item(c, g);
        };
#pragma unroll
        for (int i = 0; i < kBinRectRegs; ++i) colset(myrect[i], threadIdx.x + (int64_t)i * kBinThreads);
        for (int64_t g = threadIdx.x + (int64_t)kBinRectRegs * kBinThreads; g < K; g += kBinThreads)
          colset(rect[g], g);
        __syncthreads();
        const int32_t nl = (int32_t)min(nlong, (uint32_t)kLongMax);
        if (nl > 0) {
          run_long(nl, [&](int32_t e, int32_t c) { col_item(c, long_g[e]); });
          if (threadIdx.x == 0) nlong = 0u;
        }
        copy_masks(colmask + (int64_t)cb0 * W, nc, threadIdx.x, kBinThreads);
        __syncthreads();
      }
    }
  } else {
    // Very wide tile grids (> kLdsDiffWords tile columns): counts through global memory.
    for (int64_t i = threadIdx.x; i < T; i += kBinThreads) tile_ptr[i] = 0;
    __syncthreads();
    auto count = [&](const int4 r) {
      for (int64_t row = r.x; row <= r.y; ++row)
        for (int64_t col = r.z; col <= r.w; ++col)
          atomicAdd(reinterpret_cast<unsigned long long*>(tile_ptr + row * p.C + col), 1ull);
    };
#pragma unroll
    for (int i = 0; i < kBinRectRegs; ++i) count(myrect[i]);
    for (int64_t g = threadIdx.x + (int64_t)kBinRectRegs * kBinThreads; g < K; g += kBinThreads)
      count(rect[g]);

    __threadfence();
    __syncthreads();
    Pc = block_scan_runs<kBinThreads>(tile_ptr, T, scan_lds);
    for (int64_t t = threadIdx.x; t < T; t += kBinThreads) fill[t] = 0;
  }
  if (threadIdx.x == 0) {
    const int64_t P = (int64_t)pairs_lds;
    tile_ptr[T] = Pc;
    *num_pairs = P;
    hdr->pairs = P;
    hdr->max_span = span_lds;
    if (Pc != P) hdr->status |= GF_STATUS_COUNT_MISMATCH;
  }
}

// Emission path: rectangles, counts and tile_ptr (k_emit computes the Gaussians' constants).
__global__ __launch_bounds__(kBinThreads) void k_bin(Problem p, const float* __restrict__ mu,
                                                     const float* __restrict__ chol_raw,
                                                     int64_t* __restrict__ tile_ptr,
                                                     int64_t* __restrict__ num_pairs, uint8_t* ws,
                                                     FwdLayout L) {
  bin_body<false>(p, mu, chol_raw, nullptr, tile_ptr, num_pairs, ws, L, nullptr);
}

// ------------------------------------------------------------------------------------------
// Parallel binning (mask path).  Workgroup b < R takes tile row b: its row mask and the
// tile_ptr of its C tiles; workgroup R + c takes tile column c: its column mask.  Every
// workgroup sees every Gaussian's tile rectangle, so none waits for another:
//   tile_ptr[r*C + c] = rowbase[r] + sum_{c' < c} count(r, c'),
//   rowbase[r] = sum_g w_g * clamp(r - x_g, 0, h_g)   (g's tiles in rows before r),
// with the row's counts from a difference array over its columns.  A mask word pair is one
// wave's ballot over 64 consecutive Gaussians.  k_prep, launched before, stores each
// Gaussian's rectangle, covariance and evaluation constants (four lanes per Gaussian).
constexpr int kTilesThreads = 256;

struct PrepLoad {
  float mu0, mu1, r11, r21, r22;
};

__device__ inline PrepLoad prep_load(const float* __restrict__ mu, const float* __restrict__ chol_raw,
                                     int64_t g) {
  return PrepLoad{mu[2 * g + 0], mu[2 * g + 1], chol_raw[3 * g + 0], chol_raw[3 * g + 1], chol_raw[3 * g + 2]};
}

// d softplus / dx as torch's softplus backward: x > 20 ? 1 : e^x / (e^x + 1).  In fp32 with the
// hardware exp2, within 2e-6 relative of the exact value (the argument x log2(e) <= 28.9 is
// rounded once); the finish's gradients are held to 1e-4.
__device__ inline float softplus_grad_f32(float x) {
  if (x > 20.0f) return 1.0f;
  const float e = __builtin_amdgcn_exp2f(x * 1.44269504088896341f);
  return e / (e + 1.0f);
}

// Direct gradients (gf_backward_direct).  The chain rule from a Gaussian's six moments
// S0..S5 to its gradients (finish_body) is linear in the moments, with coefficients that depend
// only on the Gaussian's parameters.  The map is computed here in double and rounded once to
// fp32, and the backward applies it to each tile's moments before its atomics.  Output k (0:
// d_amp, 1, 2: d_mu, 3..5: d_chol_raw) is dcoef[6 g + k] . (P, Q, S4, S5), where (P, Q) is
// (S1, S2) for k = 1, 2 and (S0, S3) otherwise.  With G = h [[S3, S4], [S4, S5]],
// h = -amp norm / 2, and the det term f = h S0 (normalize), dL/dcov = -A G A + f A holds
//   c00 = -h (i00^2 S3 + 2 i00 i01 S4 + i01^2 S5) + f i00
//   c01 = -h (i00 i01 S3 + (i00 i11 + i01^2) S4 + i01 i11 S5) + f i01
//   c11 = -h (i01^2 S3 + 2 i01 i11 S4 + i11^2 S5) + f i11,
// and dL/dL = 2 [[c00 l11 + c01 l21, .], [c01 l11 + c11 l21, c11 l22]] before the softplus'.
// The Gaussian's gradient slot is cleared for the backward's atomics.  (Single fields only, whose
// mu is the mean itself: no tanh.)  cov and (l11, l22) are those the binning stored, r = chol_raw.
__device__ inline void store_dcoef(const Problem& p, GfCov cov, float l11f, float l22f, float r11, float r21,
                                   float r22, float amp, int64_t g, uint8_t* ws, const FwdLayout& L) {
  const GfRenderGeom rg = gf_render_geom(cov, p.normalize);
  const double nrm = (double)rg.norm, an = (double)amp * nrm, h = -0.5 * an;
  const double i00 = rg.i00, i01 = rg.i01, i11 = rg.i11;
  const double f = (p.normalize && gf_sqrt_rn(rg.det_f) >= GF_FLT_EPS) ? h : 0.0;
  // coefficients of (S0, S3, S4, S5) in c00, c01, c11
  const double c00[4] = {f * i00, -h * i00 * i00, -h * 2.0 * i00 * i01, -h * i01 * i01};
  const double c01[4] = {f * i01, -h * i00 * i01, -h * (i00 * i11 + i01 * i01), -h * i01 * i11};
  const double c11[4] = {f * i11, -h * i01 * i01, -h * 2.0 * i01 * i11, -h * i11 * i11};
  const double l11 = l11f, l21 = r21, l22 = l22f;
  const double sp11 = (double)softplus_grad_f32(r11), sp22 = (double)softplus_grad_f32(r22);
  double d11[4], d21[4], d22[4];
#pragma unroll
  for (int j = 0; j < 4; ++j) {
    d11[j] = 2.0 * (c00[j] * l11 + c01[j] * l21) * sp11;
    d21[j] = 2.0 * (c01[j] * l11 + c11[j] * l21);
    d22[j] = 2.0 * c11[j] * l22 * sp22;
  }
  float4* out = reinterpret_cast<float4*>(ws + L.dcoef) + 6 * g;
  out[0] = make_float4((float)nrm, 0.0f, 0.0f, 0.0f);
  out[1] = make_float4((float)(an * i00), (float)(an * i01), 0.0f, 0.0f);
  out[2] = make_float4((float)(an * i01), (float)(an * i11), 0.0f, 0.0f);
  out[3] = make_float4((float)d11[0], (float)d11[1], (float)d11[2], (float)d11[3]);
  out[4] = make_float4((float)d21[0], (float)d21[1], (float)d21[2], (float)d21[3]);
  out[5] = make_float4((float)d22[0], (float)d22[1], (float)d22[2], (float)d22[3]);
  float4* dg = reinterpret_cast<float4*>(ws + L.dgrad) + 2 * g;
  dg[0] = make_float4(0.f, 0.f, 0.f, 0.f);
  dg[1] = make_float4(0.f, 0.f, 0.f, 0.f);
}

// The Gaussians' rectangles, covariances and evaluation constants.  Up to kPrepSplitMaxK
// Gaussians, four lanes per Gaussian: the lanes of a pair each take one of the two softplus
// evaluations of the Cholesky diagonal (the longest part of a Gaussian's preparation: correctly
// rounded expf and log1pf, in double) and swap the results, and the pairs of waves 0-1 then
// store the rectangle, covariance and factor (which k_bin_tiles waits for) while those of waves
// 2-3 compute and store the evaluation constants (which only the render reads), 64 Gaussians a
// workgroup: the chain each lane runs is about half as long (cfg3's binning: 7.9 -> 7.2 us).
// Beyond that, one thread per Gaussian (cfg5, K = 4096: the same time either way, and its step
// measured 1.4 us slower with the split).  Every lane runs the same functions on the same
// inputs as one thread per Gaussian would, so the results are the same bits.  kCoef (fields
// binned in the render, K <= 256, no k_bin_tiles launch): workgroups past the preparation's
// compute the chain-rule maps, a lane pair per Gaussian likewise, beside the others rather than
// after them on each thread's dependent chain.
constexpr int64_t kPrepSplitMaxK = 2048;
constexpr int64_t kCoefPerBlock = kTilesThreads / 2;  // chain-rule maps: two lanes each
bool prep_split(const Problem& p) { return p.K <= kPrepSplitMaxK; }

// One diagonal entry per lane of a pair (lane parity `half`), swapped: the pair's Cholesky factor.
__device__ inline GfChol prep_chol_pair(const PrepLoad& in, int half) {
  const float mine = gf_activate_diag(half ? in.r22 : in.r11);
  const float other = __int_as_float(__shfl_xor(__float_as_int(mine), 1));
  GfChol Lc;
  Lc.l11 = half ? other : mine;
  Lc.l21 = in.r21;
  Lc.l22 = half ? mine : other;
  return Lc;
}

// parts: 1 the rectangle, covariance and factor, 2 the evaluation constants.
// Returns the tiles the rectangle covers (parts & 1; else 0).
__device__ inline int32_t prep_store(const Problem& p, const PrepLoad& in, const GfChol& Lc,
                                     const float* __restrict__ amp, int64_t g, uint8_t* ws, const FwdLayout& L,
                                     int parts) {
  const GfCov c = gf_cov_from_chol(Lc);
  int32_t touched = 0;
  if (parts & 1) {
    reinterpret_cast<int4*>(ws + L.rect)[g] = bin_rect(p, in.mu0, in.mu1, c, &touched);
    reinterpret_cast<float4*>(ws + L.cov)[g] = make_float4(c.s00, c.s01, c.s11, 0.0f);
    reinterpret_cast<float2*>(ws + L.lfac)[g] = make_float2(Lc.l11, Lc.l22);
  }
  if (parts & 2) {
    GaussEval v = eval_from_cov(p, in.mu0, in.mu1, c, amp[g]);
    v.gid = (int32_t)g;
    store_eval(reinterpret_cast<GaussEval*>(ws + L.eval), g, v);
  }
  return touched;
}

// kCoef (tiles binned in the render) has at most kRowsMaxK / 64 preparation workgroups, one
// WsHeader::part entry each.
static_assert(1024 / 64 <= 16, "a part entry per preparation workgroup");

template <bool kCoef, bool kSplit>
__global__ __launch_bounds__(kTilesThreads) void k_prep(Problem p, const float* __restrict__ mu,
                                                        const float* __restrict__ chol_raw,
                                                        const float* __restrict__ amp, uint8_t* ws,
                                                        FwdLayout L, int64_t* num_pairs) {
  static_assert(kSplit || !kCoef, "the chain-rule workgroups follow the split preparation");
  constexpr int64_t per = kSplit ? kTilesThreads / 4 : kTilesThreads;  // Gaussians a workgroup
  const int64_t nbp = (p.K + per - 1) / per;
  const int64_t K = live_k(p);
  const int half = threadIdx.x & 1;
  if (kCoef && (int64_t)blockIdx.x >= nbp) {
    const int64_t g = ((int64_t)blockIdx.x - nbp) * kCoefPerBlock + (threadIdx.x >> 1);
    const bool valid = g < K;
    const PrepLoad in = valid ? prep_load(mu, chol_raw, g) : PrepLoad{0.f, 0.f, 0.f, 0.f, 0.f};
    const GfChol Lc = prep_chol_pair(in, half);  // every lane takes part in the swap
    if (valid && !half)
      store_dcoef(p, gf_cov_from_chol(Lc), Lc.l11, Lc.l22, in.r11, in.r21, in.r22, amp[g], g, ws, L);
    return;
  }
  if (blockIdx.x == 0 && threadIdx.x == 0) {
    WsHeader* hdr = reinterpret_cast<WsHeader*>(ws);
    hdr->status = 0u;
    hdr->heavy = 0u;
    hdr->num_pairs = num_pairs;
  }
  if constexpr (!kSplit) {  // one thread per Gaussian
    const int64_t g = (int64_t)blockIdx.x * kTilesThreads + threadIdx.x;
    if (g < K) {
      const PrepLoad in = prep_load(mu, chol_raw, g);
      prep_store(p, in, gf_activate_cholesky(in.r11, in.r21, in.r22), amp, g, ws, L, 3);
    }
    return;
  }
  const int role = threadIdx.x >> 7;  // wave-uniform: 0 rectangle, 1 evaluation constants
  const int64_t g = (int64_t)blockIdx.x * per + ((threadIdx.x & 127) >> 1);
  const bool valid = g < K;
  const PrepLoad in = valid ? prep_load(mu, chol_raw, g) : PrepLoad{0.f, 0.f, 0.f, 0.f, 0.f};
  const GfChol Lc = prep_chol_pair(in, half);  // every lane takes part in the swap
  int32_t touched = 0;
  if (valid && !half) touched = prep_store(p, in, Lc, amp, g, ws, L, role == 0 ? 1 : 2);
  if constexpr (kCoef) {
    // the workgroup's pairs and widest rectangle for the host read-back (the pairs of a
    // workgroup are at most K * T < 2^31 where the render bins the tiles)
    __shared__ int32_t part_sum[kTilesThreads / 64], part_max[kTilesThreads / 64];
    const int lane = threadIdx.x & 63, wid = threadIdx.x >> 6;
    const int32_t sum = __builtin_amdgcn_readlane(dpp_scan_i32(touched), 63);
    int32_t most = touched;
    for (int off = 32; off > 0; off >>= 1) most = max(most, __shfl_xor(most, off));
    if (lane == 0) {
      part_sum[wid] = sum;
      part_max[wid] = most;
    }
    __syncthreads();
    if (threadIdx.x == 0) {
      int32_t ps = 0, pm = 0;
#pragma unroll
      for (int w = 0; w < kTilesThreads / 64; ++w) {
        ps += part_sum[w];
        pm = max(pm, part_max[w]);
      }
      WsHeader* hdr = reinterpret_cast<WsHeader*>(ws);
      hdr->part[blockIdx.x][0] = ps;
      hdr->part[blockIdx.x][1] = pm;
    }
  }
}

__global__ __launch_bounds__(kTilesThreads) void k_bin_tiles(Problem p, int64_t* __restrict__ tile_ptr,
                                                             int64_t* __restrict__ num_pairs, uint8_t* ws,
                                                             FwdLayout L, const float* __restrict__ chol_raw,
                                                             const float* __restrict__ amp) {
  __shared__ int32_t diff[kLdsDiffWords];  // tile-row workgroups: the row's column differences
  const int64_t K = live_k(p);
  const int32_t R = p.R, C = p.C, W = p.W;
  // every mask word is written, those of Gaussians past K as zero (in capacity mode a workspace
  // keeps the words of an earlier, larger K)
  const int64_t Kw = 32 * (int64_t)W;
  const int32_t b = (int32_t)blockIdx.x;
  const bool is_row = b < R;
  const int32_t line = is_row ? b : b - R;
  const int lane = threadIdx.x & 63;
  const int4* __restrict__ rect = reinterpret_cast<const int4*>(ws + L.rect);
  uint32_t* out = reinterpret_cast<uint32_t*>(ws + (is_row ? L.rowmask : L.colmask)) + (int64_t)line * W;
  if (is_row)
    for (int32_t i = threadIdx.x; i <= C; i += kTilesThreads) diff[i] = 0;
  __syncthreads();
  int64_t before = 0, pairs = 0;
  int32_t span = 0;  // the most tiles of one rectangle (row workgroups; the last one reports it)
  // The rectangles are loaded kBinPrefetch rounds at a time, so that the rounds do not each wait
  // for their own load (4 rounds at cfg3).
  constexpr int kBinPrefetch = 8;
  for (int64_t gb = threadIdx.x & ~63; gb < Kw; gb += kBinPrefetch * kTilesThreads) {  // wave-uniform
    int4 rr[kBinPrefetch];
#pragma unroll
    for (int i = 0; i < kBinPrefetch; ++i) {
      const int64_t g = gb + (int64_t)i * kTilesThreads + lane;
      rr[i] = g < K ? rect[g] : make_int4(0, -1, 0, -1);
    }
#pragma unroll
    for (int i = 0; i < kBinPrefetch; ++i) {
      const int64_t g0 = gb + (int64_t)i * kTilesThreads;
      if (g0 >= Kw) break;
      const int64_t g = g0 + lane;
      bool covers = false;
      if (g < K) {
        const int4 r = rr[i];
        if (is_row) {
          const int32_t h = r.y - r.x + 1, w = r.w - r.z + 1;
          before += (int64_t)w * clamp_i32(line - r.x, 0, h);
          pairs += (int64_t)w * h;
          span = max(span, w * h);
          covers = r.x <= line && line <= r.y;
          if (covers) {
            atomicAdd(diff + r.z, 1);
            atomicAdd(diff + r.w + 1, -1);  // r.w + 1 <= C
          }
        } else {
          covers = r.z <= line && line <= r.w;
        }
      }
      const uint64_t bits = __builtin_amdgcn_ballot_w64(covers);
      const int64_t w0 = g0 >> 5;  // even: words w0, w0 + 1 hold Gaussians g0 .. g0 + 63
      if (lane == 0) out[w0] = (uint32_t)bits;
      if (lane == 1 && w0 + 1 < W) out[w0 + 1] = (uint32_t)(bits >> 32);
    }
  }
  if (!is_row) {
    // The chain-rule maps of Gaussians line, line + C, ... (off the binning's critical path: the
    // column workgroups finish before the row workgroups' scans)
    const float4* cv = reinterpret_cast<const float4*>(ws + L.cov);
    const float2* lf = reinterpret_cast<const float2*>(ws + L.lfac);
    for (int64_t g = line + (int64_t)C * threadIdx.x; g < K; g += (int64_t)C * kTilesThreads) {
      const float4 c4 = cv[g];
      const float2 l = lf[g];
      GfCov c;
      c.s00 = c4.x;
      c.s01 = c4.y;
      c.s11 = c4.z;
      store_dcoef(p, c, l.x, l.y, chol_raw[3 * g + 0], chol_raw[3 * g + 1], chol_raw[3 * g + 2], amp[g], g, ws, L);
    }
    return;
  }
  __syncthreads();  // the row's differences are complete
  // tile_ptr[line*C + c] = rowbase + sum_{c' < c} diff[c'] * (c - c') = rowbase + c*D(c) - E(c),
  // with D, E the exclusive prefixes of diff[c] and c*diff[c]: one scan of two sums, with
  // rowbase and the pair total as plain sums beside it.  Thread t owns columns
  // [t*per, t*per + per).
  constexpr int kWaves = kTilesThreads / 64;
  __shared__ int64_t wsum[4][kWaves];
  __shared__ int32_t wspan[kWaves];
  const int wid = threadIdx.x >> 6;
  if (line == R - 1) {  // workgroup-uniform
    for (int off = 32; off > 0; off >>= 1) span = max(span, __shfl_xor(span, off));
    if (lane == 0) wspan[wid] = span;
  }
  const int32_t per = (C + kTilesThreads - 1) / kTilesThreads;
  const int32_t cb = (int32_t)threadIdx.x * per, ce = min(cb + per, C);
  int64_t d = 0, e = 0;
  for (int32_t c = cb; c < ce; ++c) {
    d += diff[c];
    e += (int64_t)c * diff[c];
  }
  const int64_t di = wave_inclusive_scan(d), ei = wave_inclusive_scan(e);
  const int64_t bi = wave_inclusive_scan(before), pi = wave_inclusive_scan(pairs);
  if (lane == 63) {
    wsum[0][wid] = di;
    wsum[1][wid] = ei;
    wsum[2][wid] = bi;
    wsum[3][wid] = pi;
  }
  __syncthreads();
  int64_t D = di - d, E = ei - e, Dt = 0, Et = 0, rowbase = 0, total = 0;
#pragma unroll
  for (int w = 0; w < kWaves; ++w) {
    if (w < wid) {
      D += wsum[0][w];
      E += wsum[1][w];
    }
    Dt += wsum[0][w];
    Et += wsum[1][w];
    rowbase += wsum[2][w];
    total += wsum[3][w];
  }
  int64_t* tp = tile_ptr + (int64_t)line * C;
  int32_t* heavy_list = reinterpret_cast<int32_t*>(ws + L.fill);
  for (int32_t c = cb; c < ce; ++c) {
    tp[c] = rowbase + (int64_t)c * D - E;
    D += diff[c];  // the count of tile (line, c)
    E += (int64_t)c * diff[c];
    if (p.heavy > 0 && D > p.heavy)
      heavy_list[atomicAdd(&reinterpret_cast<WsHeader*>(ws)->heavy, 1u)] = line * C + c;
  }
  if (line == R - 1 && threadIdx.x == 0) {
    const int64_t P = rowbase + (int64_t)C * Dt - Et;
    tile_ptr[(int64_t)R * C] = P;
    *num_pairs = P;
    reinterpret_cast<WsHeader*>(ws)->pairs = P;
    int32_t most = 0;
#pragma unroll
    for (int w = 0; w < kWaves; ++w) most = max(most, wspan[w]);
    reinterpret_cast<WsHeader*>(ws)->max_span = most;
    reinterpret_cast<WsHeader*>(ws)->status = P == total ? 0u : GF_STATUS_COUNT_MISMATCH;
  }
}

// ------------------------------------------------------------------------------------------
// k_emit: one wave per Gaussian; the wave's lanes walk the Gaussian's tile rectangle row-major
// and claim a slot of each tile's id segment, tile_ptr[t] + an atomic on the tile's fill count.  The order
// inside a segment is fixed afterwards by the render, which sorts each segment.

// The emission of Gaussians g0 .. g0 + 64/SG - 1 of one field by one wave, SG lanes per
// Gaussian; each lane keeps up to B slot atomics in flight before it uses their results.  With
// kEval the first lane of a Gaussian's lanes also computes its evaluation constants
// (overlapping the first atomics) and stores them (otherwise bin_body<true> did).
template <bool kEval, int SG, int B>
__device__ __forceinline__ void emit_body(const Problem& p, const float* __restrict__ mu,
                                          const float* __restrict__ amp, uint8_t* ws,
                                          const FwdLayout& L, const int64_t* __restrict__ tile_ptr,
                                          int64_t* __restrict__ ids, int64_t capacity, int64_t g0) {
  static_assert(SG >= 1 && SG <= 64 && (64 % SG) == 0, "sub-group size must divide 64");
  WsHeader* hdr = reinterpret_cast<WsHeader*>(ws);
  const int4* __restrict__ rect = reinterpret_cast<const int4*>(ws + L.rect);
  uint32_t* fill = reinterpret_cast<uint32_t*>(ws + L.fill);
  const int lane = threadIdx.x & 63;
  const int sub = lane / SG, sl = lane - sub * SG;
  const int64_t g = g0 + sub;
  if (g0 >= p.K) return;
  const bool valid = g < p.K;
  const int4 r = valid ? rect[g] : make_int4(1, 0, 1, 0);
  const int32_t w = r.w - r.z + 1;
  const int32_t n = valid ? (r.y - r.x + 1) * w : 0;
  auto tile_of = [&](int32_t l) -> int64_t {
    const int32_t dr = (int32_t)((uint32_t)l / (uint32_t)w);
    return (int64_t)(r.x + dr) * p.C + (r.z + (l - dr * w));
  };
  // Slots of pairs l = base + sl + j*SG (j < B): base from tile_ptr plus the tile's fill count.
  // The unsigned slot widens without an instruction that would wait for the atomic early.
  int64_t bases[B];
  uint32_t slots[B];
  auto claim = [&](int32_t lb) {
#pragma unroll
    for (int j = 0; j < B; ++j) {
      const int32_t l = lb + sl + j * SG;
      bases[j] = 0;
      slots[j] = 0u;
      if (l < n) {
        const int64_t t = tile_of(l);
        bases[j] = tile_ptr[t];
        slots[j] = atomicAdd(fill + t, 1u);
      }
    }
  };
  claim(0);
  if (kEval && sl == 0 && valid) {
    const float4 c4 = reinterpret_cast<const float4*>(ws + L.cov)[g];
    GfCov c;
    c.s00 = c4.x;
    c.s01 = c4.y;
    c.s11 = c4.z;
    GaussEval v = eval_from_cov(p, mu_at(p, mu, 2 * g + 0), mu_at(p, mu, 2 * g + 1), c, amp[g]);
    v.gid = (int32_t)g;
    store_eval(reinterpret_cast<GaussEval*>(ws + L.eval), g, v);
    // gf_backward_direct's gradient slot, which its reduction + finish add into (on the mask
    // path store_dcoef clears it)
    float4* dg = reinterpret_cast<float4*>(ws + L.dgrad) + 2 * g;
    dg[0] = make_float4(0.f, 0.f, 0.f, 0.f);
    dg[1] = make_float4(0.f, 0.f, 0.f, 0.f);
  }
  auto place = [&](int32_t lb) {
#pragma unroll
    for (int j = 0; j < B; ++j) {
      if (lb + sl + j * SG < n) {
        const int64_t pos = bases[j] + (int64_t)slots[j];
        if (pos < 0) {
          set_status(&hdr->status, GF_STATUS_TILE_PTR_ORDER);
        } else if (pos < capacity) {
          ids[pos] = g;
        } else {
          set_status(&hdr->status, GF_STATUS_CAPACITY);
        }
      }
    }
  };
  place(0);
  // Larger rectangles: further rounds of B*SG pairs per Gaussian while any of the wave's
  // Gaussians has pairs left.
  int32_t nmax = n;
#pragma unroll
  for (int k = 0; k < 64 / SG; ++k) nmax = max(nmax, __builtin_amdgcn_readlane(n, k * SG));
  for (int32_t lb = B * SG; lb < nmax; lb += B * SG) {
    claim(lb);
    place(lb);
  }
}

// Gaussians per emission wave: the single-field kernel uses a whole wave per Gaussian (few
// Gaussians, so latency matters); the batched one packs 4 Gaussians per wave (many Gaussians,
// so the number of waves in flight matters).
constexpr int kEmitLanesSingle = 64;
constexpr int kEmitLanesBatch = 16;

__device__ inline int wave_id() { return __builtin_amdgcn_readfirstlane((int32_t)(threadIdx.x >> 6)); }

__global__ __launch_bounds__(kEmitThreads) void k_emit(Problem p, const float* __restrict__ mu,
                                                       const float* __restrict__ amp, uint8_t* ws,
                                                       FwdLayout L, const int64_t* __restrict__ tile_ptr,
                                                       int64_t* __restrict__ ids, int64_t capacity) {
  emit_body<true, kEmitLanesSingle, 1>(
      p, mu, amp, ws, L, tile_ptr, ids, capacity,
      ((int64_t)blockIdx.x * (kEmitThreads / 64) + wave_id()) * (64 / kEmitLanesSingle));
}


// ------------------------------------------------------------------------------------------
// Canonical (ascending) order of a tile's id segment.

// Ascending bitonic sort by one workgroup, "flip" form: the first step of every merge stage
// pairs i with its mirror i ^ (k-1), later steps pair i with i ^ j, and the smaller key always
// goes to the lower index.  Indices >= n behave as +infinity and are never touched.
template <typename Key>
__device__ void bitonic_sort_ascending(Key* keys, int64_t n) {
  int64_t np = 1;
  while (np < n) np <<= 1;
  for (int64_t k = 2; k <= np; k <<= 1) {
    for (int64_t j = k >> 1; j > 0; j >>= 1) {
      const int64_t flip = (j == (k >> 1)) ? (k - 1) : j;
      for (int64_t i = threadIdx.x; i < n; i += blockDim.x) {
        const int64_t partner = i ^ flip;
        if (partner > i && partner < n) {
          const Key a = keys[i], b = keys[partner];
          if (a > b) {
            keys[i] = b;
            keys[partner] = a;
          }
        }
      }
      __syncthreads();
    }
  }
}

// Orders seg[0..n) ascending (ids are distinct values in [0, K)).  On return, if
// n <= kSortLdsKeys, lds[0..n) also holds the ordered ids.  Must be called by the whole
// workgroup; ends with a barrier.
__device__ void order_segment(int64_t* seg, int64_t n, int64_t K, int32_t* lds, int64_t* lds_small,
                              uint32_t* status) {
  const int lane = threadIdx.x & 63, wid = threadIdx.x >> 6;
  if (n <= 64) {
    // Rank sort in wave 0: each lane counts the keys smaller than its own.
    if (wid == 0) {
      const int32_t key = lane < n ? (int32_t)seg[lane] : INT32_MAX;
      int rank = 0;
      for (int j = 0; j < (int)n; ++j) rank += (__shfl(key, j, 64) < key) ? 1 : 0;
      if (lane < n) {
        seg[rank] = key;
        lds[rank] = key;
      }
    }
    __syncthreads();
    return;
  }
  if (n <= kSortLdsKeys) {
    for (int64_t i = threadIdx.x; i < n; i += blockDim.x) lds[i] = (int32_t)seg[i];
    __syncthreads();
    bitonic_sort_ascending<int32_t>(lds, n);
    for (int64_t i = threadIdx.x; i < n; i += blockDim.x) seg[i] = lds[i];
    __syncthreads();
    return;
  }
  if (K <= kBitmapMaxK) {
    // Set one bit per id, scan the popcounts, expand in order.
    const int64_t words = (K + 31) >> 5;
    uint32_t* bits = reinterpret_cast<uint32_t*>(lds);
    for (int64_t i = threadIdx.x; i < words; i += blockDim.x) bits[i] = 0u;
    __syncthreads();
    for (int64_t i = threadIdx.x; i < n; i += blockDim.x) {
      const int64_t g = seg[i];
      if (g >= 0 && g < K) atomicOr(bits + (g >> 5), 1u << (g & 31));
      else set_status(status, GF_STATUS_COUNT_MISMATCH);
    }
    __syncthreads();
    const int64_t per = (words + blockDim.x - 1) / blockDim.x;
    const int64_t wb = (int64_t)threadIdx.x * per;
    const int64_t we = wb + per < words ? wb + per : words;
    int64_t cnt = 0;
    for (int64_t w = wb; w < we; ++w) cnt += __popc(bits[w]);
    int64_t total;
    int64_t pos = block_exclusive_scan<kTileThreads>(cnt, &total, lds_small);
    if (total != n && threadIdx.x == 0) set_status(status, GF_STATUS_COUNT_MISMATCH);
    for (int64_t w = wb; w < we; ++w) {
      uint32_t m = bits[w];
      while (m) {
        const int b = __ffs(m) - 1;
        m &= m - 1;
        if (pos < n) seg[pos] = (w << 5) + b;
        ++pos;
      }
    }
    __syncthreads();
    return;
  }
  bitonic_sort_ascending<int64_t>(seg, n);
}

// Orders seg[0..n) ascending with one wave (ids are distinct values in [0, K)); keys is the
// wave's private LDS region of kWaveSortKeys int32.  On return keys[0..n) holds the ordered ids
// if n <= kWaveSortKeys.  No workgroup barriers: other waves of the workgroup are unaffected.
__device__ void order_segment_wave(int64_t* seg, int64_t n, int64_t K, int32_t* keys,
                                   uint32_t* status) {
  const int lane = threadIdx.x & 63;
  if (n <= 64) {
    // Rank sort: each lane counts the keys smaller than its own (keys broadcast by readlane).
    const int32_t key = lane < n ? (int32_t)seg[lane] : INT32_MAX;
    int rank = 0;
    for (int j = 0; j < (int)n; ++j) rank += (__builtin_amdgcn_readlane(key, j) < key) ? 1 : 0;
    if (lane < n) {
      keys[rank] = key;
      if (rank != lane) seg[rank] = key;
    }
    wave_sync();
    return;
  }
  if (n <= kWaveSortKeys) {
    for (int64_t i = lane; i < n; i += 64) keys[i] = (int32_t)seg[i];
    wave_sync();
    int64_t np = 1;
    while (np < n) np <<= 1;
    for (int64_t k = 2; k <= np; k <<= 1) {
      for (int64_t j = k >> 1; j > 0; j >>= 1) {
        const int64_t flip = (j == (k >> 1)) ? (k - 1) : j;
        for (int64_t i = lane; i < n; i += 64) {
          const int64_t partner = i ^ flip;
          if (partner > i && partner < n) {
            const int32_t a = keys[i], b = keys[partner];
            if (a > b) {
              keys[i] = b;
              keys[partner] = a;
            }
          }
        }
        wave_sync();
      }
    }
    for (int64_t i = lane; i < n; i += 64) seg[i] = keys[i];
    wave_sync();
    return;
  }
  if (K <= (int64_t)kWaveSortKeys * 32) {
    // One bit per id in LDS, popcount scan, in-order expansion.
    const int64_t words = (K + 31) >> 5;
    uint32_t* bits = reinterpret_cast<uint32_t*>(keys);
    for (int64_t i = lane; i < words; i += 64) bits[i] = 0u;
    wave_sync();
    for (int64_t i = lane; i < n; i += 64) {
      const int64_t g = seg[i];
      if (g >= 0 && g < K) atomicOr(bits + (g >> 5), 1u << (g & 31));
      else set_status(status, GF_STATUS_COUNT_MISMATCH);
    }
    wave_sync();
    const int64_t per = (words + 63) / 64;
    const int64_t wb = (int64_t)lane * per;
    const int64_t we = wb + per < words ? wb + per : words;
    int64_t cnt = 0;
    for (int64_t w = wb; w < we; ++w) cnt += __popc(bits[w]);
    int64_t pos = wave_inclusive_scan(cnt) - cnt;
    for (int64_t w = wb; w < we; ++w) {
      uint32_t m = bits[w];
      while (m) {
        const int b = __ffs(m) - 1;
        m &= m - 1;
        if (pos < n) seg[pos] = (w << 5) + b;
        ++pos;
      }
    }
    wave_sync_global();  // the caller reads seg
    return;
  }
  // In place in global memory (segments longer than kWaveSortKeys with K > 16384).
  int64_t np = 1;
  while (np < n) np <<= 1;
  for (int64_t k = 2; k <= np; k <<= 1) {
    for (int64_t j = k >> 1; j > 0; j >>= 1) {
      const int64_t flip = (j == (k >> 1)) ? (k - 1) : j;
      for (int64_t i = lane; i < n; i += 64) {
        const int64_t partner = i ^ flip;
        if (partner > i && partner < n) {
          const int64_t a = seg[i], b = seg[partner];
          if (a > b) {
            seg[i] = b;
            seg[partner] = a;
          }
        }
      }
      wave_sync_global();
    }
  }
}

// ------------------------------------------------------------------------------------------
// Forward render.

__device__ inline void tile_range(const int64_t* __restrict__ tile_ptr, int64_t t, int64_t capacity,
                                  int64_t* s, int64_t* n) {
  int64_t a = tile_ptr[t], b = tile_ptr[t + 1];
  if (a < 0) a = 0;  // (a segment never starts below the id buffer)
  if (b > capacity) b = capacity;
  if (a > b) a = b;
  *s = a;
  *n = b - a;
}

// 16x16 tiles, one wave per tile (tile blockIdx.x * 4 + wave).  Lane l covers tile row l/4,
// columns 4*(l%4)..+3.  Gaussian constants are loaded one per lane for up to 64 Gaussians at
// a time and broadcast with readlane while every lane accumulates its 4 pixels.
// Tile t (16x16) of one field by one wave.  The tile's ids come from the masks (p.W > 0: the
// set bits of rowmask[tr] & colmask[tc], in ascending order, written to the tile's segment) or
// from k_emit's segment (ordered here by a rank sort and written back where they moved).
// The 16x16 block of pixels one wave of the tile kernels handles.  16x16 tiles: tile
// idx * 4 + wave.  32x32 tiles (tile_out == tile_in == 32): tile idx, quadrant `wave` (pixel
// rows / columns 16 * (wave >> 1), 16 * (wave & 1) of the tile), all four from the tile's own
// id list.  sidx numbers the blocks for the backward's accumulator stripes.
struct SubTile {
  int64_t t;
  int32_t r0, c0;
  int32_t quad;
  int64_t sidx;
};

// 16x16 tile t as a whole (heavy-tile workgroups).
__device__ inline SubTile tile16(const Problem& p, int64_t t) {
  SubTile st;
  st.t = t;
  st.quad = 0;
  const int64_t tr = t / p.C, tc = t - (t / p.C) * p.C;
  st.r0 = (int32_t)tr * 16;
  st.c0 = (int32_t)tc * 16;
  st.sidx = t;
  return st;
}

__device__ inline SubTile sub_tile(const Problem& p, int64_t idx, int wave);

// The work of workgroup blockIdx.x in a 16x16-block tile kernel with heavy-tile workgroups:
// the first nh = (tiles k_bin_tiles listed) workgroups take one listed tile each, four waves
// sharing it (q = wave, F = 4); the rest take four tiles each in tile order, one per wave, and
// skip listed tiles.  The grid has xh workgroups beyond the one-per-four-tiles ones; xh bounds
// nh (nh > xh only when the pairs exceed the id capacity: status CAPACITY), and the workgroups
// past the tiles, at the end of the grid, return.
struct HeavyItem {
  SubTile st;
  int q, F;
};
__device__ inline HeavyItem heavy_item(const Problem& p, const int32_t* __restrict__ heavy_list,
                                       const uint32_t* heavy_count, int32_t xh, uint32_t* status) {
  HeavyItem it;
  it.q = 0;
  it.F = 1;
  const int64_t b = blockIdx.x;
  int64_t nh = 0;
  if (xh > 0) {
    const int64_t T = (int64_t)p.R * p.C;
    nh = (int64_t)*heavy_count;
    if (nh > xh) {
      if (b == 0 && threadIdx.x == 0) atomicOr(status, GF_STATUS_CAPACITY);
      nh = xh;
    }
    if (b < nh) {
      const int64_t t = heavy_list[b];
      it.st = tile16(p, t < 0 || t >= T ? T : t);  // t == T: nothing to do
      it.q = wave_id();
      it.F = kTileThreads / 64;
      return it;
    }
  }
  it.st = sub_tile(p, b - nh, wave_id());
  return it;
}

__device__ inline SubTile sub_tile(const Problem& p, int64_t idx, int wave) {
  SubTile st;
  const bool q32 = p.tile_out == 32;
  st.t = q32 ? idx : idx * 4 + wave;
  st.quad = q32 ? wave : 0;
  const int64_t tr = st.t / p.C, tc = st.t - (st.t / p.C) * p.C;
  st.r0 = (int32_t)tr * p.tile_out + 16 * (st.quad >> 1);
  st.c0 = (int32_t)tc * p.tile_in + 16 * (st.quad & 1);
  st.sidx = q32 ? idx * 4 + wave : st.t;
  return st;
}

// LDS of the 16x16 render, at namespace scope so that both instantiations of render16_body in
// one kernel share one allocation: per wave, sort / expansion keys and a chunk's constants.
__shared__ int32_t r16_wkeys[kTileThreads / 64][kWaveSortKeys];
__shared__ float4 r16_wevals[kTileThreads / 64][128];
// The row-binned render's workgroups of kRowsThreads threads (a chunk's constants per wave):
// eight tile pairs share each row binning (cfg3's step 19.8 -> 19.6 us against four; sixteen
// took 20.1 us).
constexpr int kRowsThreads = 512;
__shared__ float4 r16_rows_wevals[kRowsThreads / 64][128];

__device__ __forceinline__ void render16_body(
    const Problem& p, const float* __restrict__ row_coords, const float* __restrict__ col_coords,
    const GaussEval* __restrict__ ev, const int64_t* __restrict__ tile_ptr, int64_t* ids,
    int64_t capacity, float* __restrict__ delta, uint8_t* ws, const uint32_t* __restrict__ rowmask,
    const uint32_t* __restrict__ colmask, const SubTile& st, const int4* __restrict__ rects = nullptr,
    int64_t* __restrict__ tile_ptr_out = nullptr, int q = 0, int F = 1, float* __restrict__ blk_sq = nullptr,
    const MergedOut& mo = MergedOut{nullptr, nullptr, 1.0f}) {
  // F > 1 (heavy tiles, mask path only): the F = 4 waves of the workgroup share tile st, wave q
  // taking chunks q, q + F, ... of kHeavyChunk Gaussians; wave 0 adds the others' partial sums
  // in wave order and writes the tile.  Every wave must call it (two workgroup barriers).
  const int cs = F > 1 ? kHeavyChunk : 64;
  auto& wkeys = r16_wkeys;
  WsHeader* hdr = reinterpret_cast<WsHeader*>(ws);
  const int lane = threadIdx.x & 63;
  const int wid = __builtin_amdgcn_readfirstlane((int32_t)(threadIdx.x >> 6));
  const int64_t t = st.t;
  if (t >= (int64_t)p.R * p.C) return;
  const int32_t tr = (int32_t)(t / p.C), tc = (int32_t)(t - (t / p.C) * p.C);
  const bool write_ids = st.quad == 0 && q == 0;  // one wave of a tile writes its ids
  const int32_t pr = st.r0 + (lane >> 2), pc = st.c0 + ((lane & 3) << 2);
  // coordinates first: they do not depend on the tile's segment
  const float x = row_coords[min(pr, p.M - 1)];
  // The lane's four columns as y0 and offsets from it: z of column i is z0 + wc (y_i - y0), one
  // FMA, with y_i - y0 exact for neighbouring coordinates.
  float y0, yd[4];
  {
    float y[4];
    if (pc + 3 < p.N && ((reinterpret_cast<uintptr_t>(col_coords + pc) & 15) == 0)) {
      const float4 v = *reinterpret_cast<const float4*>(col_coords + pc);
      y[0] = v.x;
      y[1] = v.y;
      y[2] = v.z;
      y[3] = v.w;
    } else {
#pragma unroll
      for (int i = 0; i < 4; ++i) y[i] = col_coords[min(pc + i, p.N - 1)];
    }
    y0 = y[0];
#pragma unroll
    for (int i = 0; i < 4; ++i) yd[i] = y[i] - y0;
  }
  float acc[4] = {0.f, 0.f, 0.f, 0.f};
  // With clamp_quad >= 80 (or none) the clamp only floors positive-definite bases below e^-40:
  // the third loop of run_chunk leaves them at their value, a difference below e^-40 |amp| per
  // Gaussian and pixel, and saves the v_med3 of every pixel.
  const bool floor_free = !p.mask_clamp;
  auto accumulate_free = [&](const GaussEval& u) {
    const float dx = x - u.mu0;
    const float a = u.wa * dx;
    const float z0 = fmaf(u.wc, y0 - u.mu1, u.wb * dx);
    const float A = a * a;
#pragma unroll
    for (int i = 0; i < 4; ++i) {
      const float z = i == 0 ? z0 : fmaf(u.wc, yd[i], z0);
      acc[i] = fmaf(u.w, __builtin_amdgcn_exp2f(-fmaf(z, z, A)), acc[i]);
    }
  };
  auto accumulate = [&](const GaussEval& u, auto general) {
    const float dx = x - u.mu0;
    const float a = u.wa * dx;
    const float z0 = fmaf(u.wc, y0 - u.mu1, u.wb * dx);
    if (general && u.gen != 0.0f) {  // indefinite form (uniform: u is broadcast)
      const float nA = -(a * a);
#pragma unroll
      for (int i = 0; i < 4; ++i) {
        const float z = i == 0 ? z0 : fmaf(u.wc, yd[i], z0);
        acc[i] = fmaf(u.w, basis_q(p, fmaf(z, z, nA)), acc[i]);
      }
      return;
    }
    const float A = a * a;
#pragma unroll
    for (int i = 0; i < 4; ++i) {
      const float z = i == 0 ? z0 : fmaf(u.wc, yd[i], z0);
      // definite forms as in accumulate_free whenever the floor is dropped, so that a pixel's
      // value does not depend on which loop its chunk took
      const float e = floor_free ? __builtin_amdgcn_exp2f(-fmaf(z, z, A)) : basis_w(p, A, z);
      acc[i] = fmaf(u.w, e, acc[i]);
    }
  };
  // Gaussians 0 .. nj-1 of a chunk (lane j holds Gaussian j), staged in the wave's LDS and
  // read back in order with broadcast loads (two ds_read_b128 per Gaussian instead of a
  // v_readlane per constant); one ballot per chunk picks the loop that handles general-form
  // Gaussians.
  auto& wevals = r16_wevals;
  float4* ew = wevals[wid];
  auto run_chunk = [&](const GaussEval& my, int nj) {
    // two arrays of 64 float4 (conflict-free writes, broadcast reads)
    ew[lane] = make_float4(my.mu0, my.mu1, my.wa, my.wb);
    ew[64 + lane] = make_float4(my.wc, my.w, __int_as_float(my.gid), my.gen);
    wave_sync();
    auto at = [&](int j) {
      const float4 a = ew[j], b = ew[64 + j];
      GaussEval u;
      u.mu0 = a.x;
      u.mu1 = a.y;
      u.wa = a.z;
      u.wb = a.w;
      u.wc = b.x;
      u.w = b.y;
      u.gid = __float_as_int(b.z);
      u.gen = b.w;
      return u;
    };
    if (__builtin_amdgcn_ballot_w64(lane < nj && my.gen != 0.0f) == 0) {
      if (floor_free)
        for (int j = 0; j < nj; ++j) accumulate_free(at(j));
      else
        for (int j = 0; j < nj; ++j) accumulate(at(j), std::false_type{});
    } else {
      for (int j = 0; j < nj; ++j) accumulate(at(j), std::true_type{});
    }
    wave_sync();  // every lane has read the slots before the next chunk rewrites them
  };
  int64_t s, n;
  if (p.W > 0) {
    // The tile's segment [s, s + count); ids past the capacity are not stored.
    int64_t count;
    const uint32_t* own = nullptr;
    if (rects) {
      // Tiles binned here (tiles_in_render): the tile's mask words, one ballot per 64
      // Gaussians, into the wave's LDS, its count, and its segment start in closed form -- the
      // pairs of every Gaussian in earlier tiles, row-major:
      //   w_g * clamp(tr - x_g, 0, h_g) + [x_g <= tr <= y_g] * clamp(tc - z_g, 0, w_g).
      __shared__ uint32_t wmask[kTileThreads / 64][kMaskMaxK / 32];
      uint32_t* mw = wmask[wid];
      int64_t before = 0, cnt = 0;
      int32_t span = 0;  // the most tiles of one rectangle, for the workspace header
      constexpr int kPre = 4;  // rounds of rectangle loads in flight (K <= 256: all of them)
      // every mask word of the tile is written, those of Gaussians past the live K as zero
      const int64_t Kl = live_k(p), Kw = 32 * (int64_t)p.W;
      for (int64_t gb = 0; gb < Kw; gb += kPre * 64) {
        int4 rr[kPre];
#pragma unroll
        for (int i = 0; i < kPre; ++i) {
          const int64_t g = gb + 64 * i + lane;
          rr[i] = g < Kl ? rects[g] : make_int4(0, -1, 0, -1);
        }
#pragma unroll
        for (int i = 0; i < kPre; ++i) {
          const int64_t g0 = gb + 64 * i;
          if (g0 >= Kw) break;
          const int64_t g = g0 + lane;
          bool covers = false;
          if (g < Kl) {
            const int4 r = rr[i];
            const int32_t h = r.y - r.x + 1, wd = r.w - r.z + 1;
            const bool in_row = r.x <= tr && tr <= r.y;
            before += (int64_t)wd * clamp_i32(tr - r.x, 0, h) + (in_row ? clamp_i32(tc - r.z, 0, wd) : 0);
            span = max(span, wd * h);
            covers = in_row && r.z <= tc && tc <= r.w;
          }
          const uint64_t bits = __builtin_amdgcn_ballot_w64(covers);
          cnt += __popcll(bits);
          const int32_t w0 = (int32_t)(g0 >> 5);
          if (lane == 0) mw[w0] = (uint32_t)bits;
          if (lane == 1 && w0 + 1 < p.W) mw[w0 + 1] = (uint32_t)(bits >> 32);
        }
      }
      s = readlane_i64(wave_inclusive_scan(before), 63);
      count = cnt;
      const int64_t T = (int64_t)p.R * p.C;
      if (write_ids && t == T - 1) {  // wave-uniform
        for (int off = 32; off > 0; off >>= 1) span = max(span, __shfl_xor(span, off));
        if (lane == 0) {
          hdr->pairs = s + count;
          hdr->max_span = span;
        }
      }
      if (write_ids && lane == 0) {
        tile_ptr_out[t] = s;
        if (t == T - 1) {
          tile_ptr_out[T] = s + count;
          *hdr->num_pairs = s + count;
        }
      }
      wave_sync();
      own = mw;
    } else {
      s = tile_ptr[t];
      count = tile_ptr[t + 1] - s;
      if (F == 1 && p.heavy > 0 && count > p.heavy) return;  // a heavy-tile workgroup's
    }
    // ids are written to [s, s + room): none for a segment below the id buffer or reversed
    const int64_t room = s < 0 ? 0 : capacity - s < count ? (capacity - s > 0 ? capacity - s : 0) : count;
    if ((s < 0 || count < 0) && write_ids && lane == 0) set_status(&hdr->status, GF_STATUS_TILE_PTR_ORDER);
    const uint32_t* rm = rowmask + (int64_t)tr * p.W;
    const uint32_t* cm = colmask + (int64_t)tc * p.W;
    int32_t* keys = wkeys[wid];
    int64_t done = 0;
    for (int32_t w0 = 0; w0 < p.W; w0 += 64) {
      const int32_t w = w0 + lane;
      const uint32_t m = w < p.W ? (own ? own[w] : (rm[w] & cm[w])) : 0u;
      const int32_t cnt = __popc(m);
      const int32_t inc = dpp_scan_i32(cnt);
      const int32_t tot = __builtin_amdgcn_readlane(inc, 63);
      // Expand the set bits in order, kWaveSortKeys positions at a time.
      for (int32_t base = 0; base < tot; base += kWaveSortKeys) {
        uint32_t mm = m;
        int32_t pos = inc - cnt;
        while (mm != 0u && pos < base + kWaveSortKeys) {
          const int32_t bit = __builtin_ctz(mm);
          mm &= mm - 1u;
          if (pos >= base) keys[pos - base] = (w << 5) + bit;
          ++pos;
        }
        wave_sync();
        const int32_t nwin = min(kWaveSortKeys, tot - base);
        if (write_ids) {
          for (int32_t j = lane; j < nwin; j += 64) {
            const int64_t slot = done + j;
            if (slot < room) ids[s + slot] = keys[j];
          }
        }
        for (int32_t j0 = q * cs; j0 < nwin; j0 += F * cs) {
          const int nj = min(cs, nwin - j0);
          GaussEval my = zero_eval();
          if (lane < nj) my = load_eval(ev, keys[j0 + lane]);
          run_chunk(my, nj);
        }
        done += nwin;
        wave_sync();
      }
    }
    if (lane == 0 && write_ids) {
      if (done != count) set_status(&hdr->status, GF_STATUS_COUNT_MISMATCH);
      if (room < count) set_status(&hdr->status, GF_STATUS_CAPACITY);
    }
    n = 0;  // rendered
  } else {
    tile_range(tile_ptr, t, capacity, &s, &n);
  }
  if (n > 0 && n <= 64) {
    // Rank sort of the ids (emission order); each lane gathers its Gaussian's constants while
    // the ranks are computed, then they follow their id to lane `rank` (ds_permute).
    GaussEval my = zero_eval();
    int32_t key = INT32_MAX;
    if (lane < n) {
      key = (int32_t)ids[s + lane];
      if (key >= 0 && key < p.K) my = load_eval(ev, key);
    }
    int rank = 0;
    for (int j = 0; j < (int)n; ++j) rank += (__builtin_amdgcn_readlane(key, j) < key) ? 1 : 0;
    const int addr = rank << 2;
    GaussEval srt;
    srt.mu0 = __int_as_float(__builtin_amdgcn_ds_permute(addr, __float_as_int(my.mu0)));
    srt.mu1 = __int_as_float(__builtin_amdgcn_ds_permute(addr, __float_as_int(my.mu1)));
    srt.wa = __int_as_float(__builtin_amdgcn_ds_permute(addr, __float_as_int(my.wa)));
    srt.wb = __int_as_float(__builtin_amdgcn_ds_permute(addr, __float_as_int(my.wb)));
    srt.wc = __int_as_float(__builtin_amdgcn_ds_permute(addr, __float_as_int(my.wc)));
    srt.w = __int_as_float(__builtin_amdgcn_ds_permute(addr, __float_as_int(my.w)));
    srt.gid = __builtin_amdgcn_ds_permute(addr, key);  // key == my.gid for a valid id
    srt.gen = __int_as_float(__builtin_amdgcn_ds_permute(addr, __float_as_int(my.gen)));
    if (lane < n) {
      if (srt.gid < 0 || srt.gid >= p.K) set_status(&hdr->status, GF_STATUS_COUNT_MISMATCH);
      if (srt.gid != key) ids[s + lane] = srt.gid;  // lanes whose id moved
    }
    run_chunk(srt, (int)n);
  } else if (n > 64) {
    int64_t* seg = ids + s;
    int32_t* keys = wkeys[wid];
    order_segment_wave(seg, n, p.K, keys, &hdr->status);
    for (int64_t j0 = 0; j0 < n; j0 += 64) {
      const int nj = (int)((n - j0) < 64 ? (n - j0) : 64);
      GaussEval my = zero_eval();
      if (lane < nj) {
        const int64_t g = (n <= kWaveSortKeys) ? (int64_t)keys[j0 + lane] : seg[j0 + lane];
        if (g >= 0 && g < p.K) {
          my = load_eval(ev, g);
        } else {
          set_status(&hdr->status, GF_STATUS_COUNT_MISMATCH);  // internal mismatch only
        }
      }
      run_chunk(my, nj);
    }
  }
  if (F > 1) {
    if (wid != 0) ew[lane] = make_float4(acc[0], acc[1], acc[2], acc[3]);
    __syncthreads();
    if (wid == 0) {
      for (int w = 1; w < F; ++w) {
        const float4 v = wevals[w][lane];
        acc[0] += v.x;
        acc[1] += v.y;
        acc[2] += v.z;
        acc[3] += v.w;
      }
    }
    __syncthreads();  // the partial sums are read before the slots are reused
    if (wid != 0) return;
  }
  if (blk_sq) {  // the block's sum of squares (the layer's ||delta-W||, reduced by k_batch_read)
    float sq = 0.f;
    if (pr < p.M) {
#pragma unroll
      for (int i = 0; i < 4; ++i)
        if (pc + i < p.N) sq = fmaf(acc[i], acc[i], sq);
    }
    sq = dpp_scan_f32(sq);
    if (lane == 63) blk_sq[st.sidx] = sq;
  }
  if (pr < p.M) store_row4(p, delta, mo, pr, pc, acc);
}

// Two horizontally adjacent 16x16 tiles of one field by one wave, on the mask path (p.W > 0):
// tiles (tr, tc) and (tr, tc + 1), the second absent when tc + 1 == p.C.  Lane l covers tile row
// l/4, columns 4*(l%4)..+3 of both tiles.  The wave expands the union of the two tiles' mask
// bits once and stages each Gaussian of the union once, with a zero amplitude for a tile that
// does not list it: for a definite form the basis is finite, so fma(0, e, acc) == acc exactly,
// and indefinite forms are skipped per tile.  Every pixel thus sums its own tile's Gaussians in
// ascending id order with the arithmetic of render16_body, bit for bit, while the per-tile
// work (mask loads, scans, gathers, waits) is shared by twice the pixels.  Each tile's ids are
// written to its own segment chunk by chunk.
constexpr int32_t kPairInA = 1 << 14, kPairInB = 1 << 15, kPairIdMask = kPairInA - 1;  // ids < kMaskMaxK
static_assert(kMaskMaxK <= kPairInA, "pair keys hold the id below the tile flags");

// A tile row binned by its render workgroup (k_render16x2_rows): the row's Gaussians in
// ascending id order, each with its first and last tile column, the pairs of the tile rows
// above, and where the row's segment starts go.
struct RowBin {
  const int2* list;          // LDS: (id, first column | last column << 16)
  int32_t n;                 // entries
  int64_t base;              // pairs in tile rows 0 .. tr - 1
  int32_t span;              // the most tiles one rectangle covers (the field's)
  int64_t* tile_ptr_out;     // tile_ptr, written for the wave's tiles (and [T] by tile T - 1's wave)
};

template <bool kSkipHalves, bool kRows = false>
__device__ __forceinline__ void render16x2_body(
    const Problem& p, const float* __restrict__ row_coords, const float* __restrict__ col_coords,
    const GaussEval* __restrict__ ev, const int64_t* __restrict__ tile_ptr, int64_t* __restrict__ ids,
    int64_t capacity, float* __restrict__ delta, uint8_t* ws, const uint32_t* __restrict__ rowmask,
    const uint32_t* __restrict__ colmask, int32_t tr, int32_t tc, float* __restrict__ blk_sq,
    const MergedOut& mo = MergedOut{nullptr, nullptr, 1.0f}, uint32_t skip = 0u,
    const RowBin& rb = RowBin{nullptr, 0, 0, 0, nullptr}) {
  // skip: bit 0 leaves tile A, bit 1 tile B to another workgroup (a heavy tile): no Gaussians,
  // ids, checks or stores of that tile here.  kRows: the segments and the Gaussians come from
  // the workgroup's row list rb (tile_ptr, rowmask and colmask are not read), and the wave
  // writes its tiles' segment starts.
  WsHeader* hdr = reinterpret_cast<WsHeader*>(ws);
  const int lane = threadIdx.x & 63;
  const int wid = __builtin_amdgcn_readfirstlane((int32_t)(threadIdx.x >> 6));
  const bool has_a = (skip & 1u) == 0u;
  const bool has_b = tc + 1 < p.C && (skip & 2u) == 0u;
  const int64_t ta = (int64_t)tr * p.C + tc;
  const int32_t pr = tr * 16 + (lane >> 2);
  const int32_t pc0 = tc * 16 + ((lane & 3) << 2);
  const float x = row_coords[min(pr, p.M - 1)];
  float y0[2], yd[2][4];
  // both tiles' columns inside the matrix from a 16-byte aligned base (the same in every lane):
  // every lane's four columns are one aligned float4, without per-lane tests (the row-binned
  // kernel keeps those, as in the stores below)
  const bool cols4 = !kRows && (tc + 2) * 16 <= p.N && (reinterpret_cast<uintptr_t>(col_coords) & 15) == 0;
#pragma unroll
  for (int h = 0; h < 2; ++h) {
    const int32_t pc = pc0 + 16 * h;
    float y[4];
    if (cols4 || (pc + 3 < p.N && ((reinterpret_cast<uintptr_t>(col_coords + pc) & 15) == 0))) {
      const float4 v = *reinterpret_cast<const float4*>(col_coords + pc);
      y[0] = v.x;
      y[1] = v.y;
      y[2] = v.z;
      y[3] = v.w;
    } else {
#pragma unroll
      for (int i = 0; i < 4; ++i) y[i] = col_coords[min(pc + i, p.N - 1)];
    }
    y0[h] = y[0];
#pragma unroll
    for (int i = 0; i < 4; ++i) yd[h][i] = y[i] - y[0];
  }
  float acc[2][4] = {{0.f, 0.f, 0.f, 0.f}, {0.f, 0.f, 0.f, 0.f}};
  const bool floor_free = !p.mask_clamp;
  // The two segments are adjacent: [sa, sb) and [sb, se).
  int64_t sa, sb, se;
  int32_t key0 = 0;  // kRows: the first chunk (row entries 0 .. 63)
  bool keep0 = false;
  GaussEval pre0 = zero_eval();
  if constexpr (kRows) {
    // Segment start of tile A in closed form, the pairs of every Gaussian in earlier tiles
    // (row-major): the rows above (rb.base) plus clamp(tc - first, 0, width) over the row's
    // Gaussians; tile B starts after tile A's count.
    // (32-bit sums: before <= n * C < 2^25, counts <= n <= 1024 in two 16-bit halves).  The
    // first 64 entries' keys and constants are kept for the first chunk: the constants' gather
    // overlaps the sums.
    int32_t before = 0, nab = 0;
    for (int32_t j = lane; j < rb.n; j += 64) {
      const int2 e = rb.list[j];
      const int32_t z = e.y & 0xffff, w = e.y >> 16;
      const bool ia = z <= tc && tc <= w, ib = has_b && z <= tc + 1 && tc + 1 <= w;
      before += clamp_i32(tc - z, 0, w - z + 1);
      nab += (ia ? 1 : 0) + (ib ? 0x10000 : 0);
      if (j < 64) {
        keep0 = ia || ib;
        key0 = e.x | (ia ? kPairInA : 0) | (ib ? kPairInB : 0);
        if (keep0) pre0 = load_eval(ev, e.x);
      }
    }
    before = __builtin_amdgcn_readlane(dpp_scan_i32(before), 63);
    nab = __builtin_amdgcn_readlane(dpp_scan_i32(nab), 63);
    const int32_t na = nab & 0xffff, nb = nab >> 16;
    sa = rb.base + before;
    sb = sa + na;
    se = sb + nb;
    const int64_t T = (int64_t)p.R * p.C;
    const int64_t last = has_b ? ta + 1 : ta;
    if (lane == 0) {
      rb.tile_ptr_out[ta] = sa;
      if (has_b) rb.tile_ptr_out[ta + 1] = sb;
      if (last == T - 1) {
        rb.tile_ptr_out[T] = se;
        *hdr->num_pairs = se;
        hdr->pairs = se;
        hdr->max_span = rb.span;
      }
    }
  } else {
    sa = tile_ptr[ta];
    sb = tile_ptr[ta + 1];
    se = has_b ? tile_ptr[ta + 2] : sb;
  }
  const int64_t cnt_a = has_a ? sb - sa : 0, cnt_b = se - sb;
  // ids are written to [s, s + room): none for a segment below the id buffer or reversed
  auto room_of = [&](int64_t s, int64_t count) {
    return s < 0 ? 0 : capacity - s < count ? (capacity - s > 0 ? capacity - s : 0) : count;
  };
  const int64_t room_a = room_of(sa, cnt_a), room_b = room_of(sb, cnt_b);
  if ((sa < 0 || cnt_a < 0 || cnt_b < 0) && lane == 0) set_status(&hdr->status, GF_STATUS_TILE_PTR_ORDER);
  int32_t* keys = r16_wkeys[kRows ? 0 : wid];  // (not used by kRows)
  float4* ew = kRows ? r16_rows_wevals[wid] : r16_wevals[wid];

  // One chunk of nj <= 64 union Gaussians (key kf in the active lanes, ascending with the lane):
  // each tile's ids go to its segment at the lane's rank among the chunk's keys of that tile;
  // the active lane of rank j stages Gaussian j (constants, each tile's amplitude, flags: 1 tile
  // A, 2 tile B, 4 indefinite form) and every lane adds its 8 pixels.
  int32_t done_a = 0, done_b = 0;  // ids of each tile so far (< K)
  auto run_chunk = [&](int32_t kf, bool active, int nj, const GaussEval* given = nullptr) {
    const bool in_a = active && (kf & kPairInA) != 0, in_b = active && (kf & kPairInB) != 0;
    const uint64_t bal_a = __builtin_amdgcn_ballot_w64(in_a), bal_b = __builtin_amdgcn_ballot_w64(in_b);
    const int32_t id = kf & kPairIdMask;
    if (in_a) {
      const int32_t r = done_a + (int32_t)__builtin_amdgcn_mbcnt_hi((uint32_t)(bal_a >> 32),
                                                                    __builtin_amdgcn_mbcnt_lo((uint32_t)bal_a, 0u));
      if (r < room_a) ids[sa + r] = id;
    }
    if (in_b) {
      const int32_t r = done_b + (int32_t)__builtin_amdgcn_mbcnt_hi((uint32_t)(bal_b >> 32),
                                                                    __builtin_amdgcn_mbcnt_lo((uint32_t)bal_b, 0u));
      if (r < room_b) ids[sb + r] = id;
    }
    done_a += __popcll(bal_a);
    done_b += __popcll(bal_b);
    GaussEval my = zero_eval();
    if (active) my = given ? *given : load_eval(ev, id);
    const int32_t fl = (in_a ? 1 : 0) | (in_b ? 2 : 0) | (my.gen != 0.0f ? 4 : 0);
    // two arrays of 64 float4 (conflict-free writes, broadcast reads)
    // (the mask path's active lanes are 0 .. nj - 1, its own ranks)
    int si = lane;
    if constexpr (kRows) {
      const uint64_t bal = __builtin_amdgcn_ballot_w64(active);
      si = (int)__builtin_amdgcn_mbcnt_hi((uint32_t)(bal >> 32), __builtin_amdgcn_mbcnt_lo((uint32_t)bal, 0u));
    }
    if (!kRows || active) {
      ew[si] = make_float4(my.mu0, my.mu1, my.wa, my.wb);
      ew[64 + si] = make_float4(my.wc, in_a ? my.w : 0.0f, in_b ? my.w : 0.0f, __int_as_float(fl));
    }
    const bool general = __builtin_amdgcn_ballot_w64((fl & 4) != 0) != 0;
    wave_sync();
    // kSkipHalves (batches): a Gaussian of one tile only (a third of the union at cfg4) skips the
    // other tile's half: the flags are the same in every lane (one Gaussian at a time), so the
    // branch is scalar, and skipping the zero-amplitude half leaves acc as the no-op fma would.
    // Single fields of larger Gaussians (cfg3: nearly all in both tiles) do not repay the
    // readfirstlane and branches.
    auto definite = [&](const float4& a, const float4& b, auto free_form) {
      const int32_t f = kSkipHalves ? __builtin_amdgcn_readfirstlane(__float_as_int(b.w)) : 3;
      const float dx = x - a.x;
      const float aa = a.z * dx;
      const float bb = a.w * dx;
      const float A = aa * aa;
      // kSkipHalves: the slot's per-tile constants in registers before the per-tile branches,
      // one LDS read of the slot and one address, not a read and an address per branch
      const float mu1 = a.y, wc = b.x, wab[2] = {b.y, b.z};
      if constexpr (kSkipHalves) __asm__ volatile("" ::"v"(mu1), "v"(wc), "v"(wab[0]), "v"(wab[1]));
#pragma unroll
      for (int h = 0; h < 2; ++h) {
        if ((f & (1 << h)) == 0) continue;
        const float wh = wab[h];
        const float z0 = fmaf(wc, y0[h] - mu1, bb);
#pragma unroll
        for (int i = 0; i < 4; ++i) {
          const float z = i == 0 ? z0 : fmaf(wc, yd[h][i], z0);
          const float e = free_form ? __builtin_amdgcn_exp2f(-fmaf(z, z, A)) : basis_w(p, A, z);
          acc[h][i] = fmaf(wh, e, acc[h][i]);
        }
      }
    };
    if (!general) {
      if (floor_free)
        for (int j = 0; j < nj; ++j) definite(ew[j], ew[64 + j], std::true_type{});
      else
        for (int j = 0; j < nj; ++j) definite(ew[j], ew[64 + j], std::false_type{});
    } else {
      for (int j = 0; j < nj; ++j) {
        const float4 a = ew[j], b = ew[64 + j];
        const int32_t f = __builtin_amdgcn_readfirstlane(__float_as_int(b.w));
        if ((f & 4) == 0) {
          if (floor_free)
            definite(a, b, std::true_type{});
          else
            definite(a, b, std::false_type{});
          continue;
        }
        // indefinite form (q' = z^2 - a^2), only on the tiles that list it
        const float dx = x - a.x;
        const float aa = a.z * dx;
        const float nA = -(aa * aa);
        const float bb = a.w * dx;
#pragma unroll
        for (int h = 0; h < 2; ++h) {
          if ((f & (1 << h)) == 0) continue;
          const float wh = h == 0 ? b.y : b.z;
          const float z0 = fmaf(b.x, y0[h] - a.y, bb);
#pragma unroll
          for (int i = 0; i < 4; ++i) {
            const float z = i == 0 ? z0 : fmaf(b.x, yd[h][i], z0);
            acc[h][i] = fmaf(wh, basis_q(p, fmaf(z, z, nA)), acc[h][i]);
          }
        }
      }
    }
    wave_sync();  // every lane has read the slots before the next chunk rewrites them
  };

  if constexpr (kRows) {
    // 64 row Gaussians at a time: those in tile A or B are a chunk, staged in id order
    {
      const uint64_t bal = __builtin_amdgcn_ballot_w64(keep0);
      if (bal != 0ull) run_chunk(key0, keep0, __popcll(bal), &pre0);  // wave-uniform
    }
    for (int32_t j0 = 64; j0 < rb.n; j0 += 64) {
      const int32_t j = j0 + lane;
      int32_t kf = 0;
      bool keep = false;
      if (j < rb.n) {
        const int2 e = rb.list[j];
        const int32_t z = e.y & 0xffff, w = e.y >> 16;
        const bool ia = z <= tc && tc <= w, ib = has_b && z <= tc + 1 && tc + 1 <= w;
        keep = ia || ib;
        kf = e.x | (ia ? kPairInA : 0) | (ib ? kPairInB : 0);
      }
      const uint64_t bal = __builtin_amdgcn_ballot_w64(keep);
      if (bal != 0ull) run_chunk(kf, keep, __popcll(bal));  // wave-uniform
    }
  }
  const uint32_t* rm = kRows ? nullptr : rowmask + (int64_t)tr * p.W;
  const uint32_t* cma = kRows ? nullptr : colmask + (int64_t)tc * p.W;
  const uint32_t* cmb = kRows ? nullptr : cma + p.W;  // read only when has_b
  for (int32_t w0 = 0; !kRows && w0 < p.W; w0 += 64) {
    const int32_t w = w0 + lane;
    uint32_t ma = 0u, mb = 0u;
    if (w < p.W) {
      const uint32_t r = rm[w];
      if (has_a) ma = r & cma[w];
      if (has_b) mb = r & cmb[w];
    }
    const uint32_t u = ma | mb;
    const int32_t cu = __popc(u);
    const int32_t inc_u = dpp_scan_i32(cu);
    const int32_t tot_u = __builtin_amdgcn_readlane(inc_u, 63);
    for (int32_t base = 0; base < tot_u; base += kWaveSortKeys) {
      uint32_t mm = u;
      int32_t pos = inc_u - cu;
      while (mm != 0u && pos < base + kWaveSortKeys) {
        const int32_t bit = __builtin_ctz(mm);
        mm &= mm - 1u;
        if (pos >= base)
          keys[pos - base] = ((w << 5) + bit) | (int32_t)(((ma >> bit) & 1u) << 14) | (int32_t)(((mb >> bit) & 1u) << 15);
        ++pos;
      }
      wave_sync();
      const int32_t nwin = min(kWaveSortKeys, tot_u - base);
      for (int32_t j0 = 0; j0 < nwin; j0 += 64) {
        const int nj = min(64, nwin - j0);
        run_chunk(lane < nj ? keys[j0 + lane] : 0, lane < nj, nj);
      }
      wave_sync();
    }
  }
  if (lane == 0) {
    if (done_a != cnt_a || done_b != cnt_b) set_status(&hdr->status, GF_STATUS_COUNT_MISMATCH);
    if (room_a < cnt_a || room_b < cnt_b) set_status(&hdr->status, GF_STATUS_CAPACITY);
  }
#pragma unroll
  for (int h = 0; h < 2; ++h) {
    if (h == 0 && !has_a) continue;
    if (h == 1 && !has_b) break;
    const int32_t pc = pc0 + 16 * h;
    const bool tile_inner = (tr + 1) * 16 <= p.M && (tc + h + 1) * 16 <= p.N;  // wave-uniform
    if (blk_sq) {  // as in render16_body
      float sq = 0.f;
      if (tile_inner) {
        // a tile inside the matrix (the same answer in every lane: a scalar branch) sums its
        // pixels without the per-pixel bounds selects, in the same order
#pragma unroll
        for (int i = 0; i < 4; ++i) sq = fmaf(acc[h][i], acc[h][i], sq);
      } else if (pr < p.M) {
#pragma unroll
        for (int i = 0; i < 4; ++i)
          if (pc + i < p.N) sq = fmaf(acc[h][i], acc[h][i], sq);
      }
      sq = dpp_scan_f32(sq);
      if (lane == 63) blk_sq[ta + h] = sq;
    }
    // (the row-binned single-field kernel keeps the per-lane test: there the scalar one measured
    // no faster, 8.44 against 8.36 us at cfg3 over three A/B pairs, where batches gained 3%)
    if (pr < p.M) store_row4(p, delta, mo, pr, pc, acc[h], !kRows && tile_inner);
  }
}

// Single 16x16 fields on the mask path without heavy tiles: a pair of horizontally adjacent
// tiles a wave, four pairs (R x ceil(C / 2), row-major) a workgroup.
__global__ __launch_bounds__(kTileThreads) void k_render16x2(
    Problem p, const float* __restrict__ row_coords, const float* __restrict__ col_coords,
    const GaussEval* __restrict__ ev, const int64_t* __restrict__ tile_ptr, int64_t* ids, int64_t capacity,
    float* __restrict__ delta, uint8_t* ws, const uint32_t* __restrict__ rowmask,
    const uint32_t* __restrict__ colmask) {
  const int32_t cp = (p.C + 1) / 2;
  const int64_t pi = (int64_t)blockIdx.x * (kTileThreads / 64) + wave_id();
  if (pi >= (int64_t)p.R * cp) return;
  const int32_t tr = (int32_t)pi / cp, tc = 2 * ((int32_t)pi - tr * cp);
  render16x2_body<false>(p, row_coords, col_coords, ev, tile_ptr, ids, capacity, delta, ws, rowmask, colmask, tr,
                         tc, nullptr);
}

// The row binning (bin_tile_row) lists at most kRowsMaxK Gaussians a tile row.
constexpr int64_t kRowsMaxK = 1024;

// LDS of a workgroup's tile-row binning (up to kRowsThreads / 64 waves).
struct RowLds {
  int2 list[kRowsMaxK];
  uint64_t bits[kRowsMaxK / 64];
  int32_t before[kRowsThreads / 64];
  int32_t span[kRowsThreads / 64];
};

// Tile row tr of a field binned by the whole workgroup (every thread calls it; two barriers):
// the row's Gaussians in rl.list in ascending id order, the pairs of the rows above and, in the
// grid's last workgroup (which holds tile T - 1), the widest rectangle.
template <int kThreads>
__device__ inline RowBin bin_tile_row(const Problem& p, const int4* __restrict__ rects, int32_t tr, RowLds& rl,
                                      int64_t* tile_ptr_out) {
  constexpr int kRowsPer = (int)(kRowsMaxK / kThreads);  // rectangles a thread
  constexpr int kWaves = kThreads / 64;
  const int lane = threadIdx.x & 63;
  const int wid = __builtin_amdgcn_readfirstlane((int32_t)(threadIdx.x >> 6));
  const int64_t Kl = live_k(p);
  int4 rr[kRowsPer];
#pragma unroll
  for (int i = 0; i < kRowsPer; ++i) {
    const int64_t g = (int64_t)kThreads * i + threadIdx.x;
    rr[i] = g < Kl ? rects[g] : make_int4(0, -1, 0, -1);
  }
  // (32-bit sums: the pairs of the rows above are at most P <= K * T < 2^31, rows_fit)
  int32_t before = 0, span = 0;
  const bool last_wg = blockIdx.x == gridDim.x - 1;  // tile T - 1's: writes the widest rectangle
  uint64_t bits[kRowsPer];
#pragma unroll
  for (int i = 0; i < kRowsPer; ++i) {
    const int4 r = rr[i];
    const bool live = (int64_t)kThreads * i + threadIdx.x < Kl;
    const int32_t h = r.y - r.x + 1, wd = r.w - r.z + 1;
    const bool in_row = live && r.x <= tr && tr <= r.y;
    if (live) {
      before += wd * clamp_i32(tr - r.x, 0, h);
      if (last_wg) span = max(span, wd * h);
    }
    bits[i] = __builtin_amdgcn_ballot_w64(in_row);
    if (lane == 0) rl.bits[i * kWaves + wid] = bits[i];
  }
  before = __builtin_amdgcn_readlane(dpp_scan_i32(before), 63);
  if (last_wg)
    for (int off = 32; off > 0; off >>= 1) span = max(span, __shfl_xor(span, off));
  if (lane == 0) {
    rl.before[wid] = before;
    rl.span[wid] = span;
  }
  __syncthreads();
  // Word q = i * kWaves + wave holds Gaussians 64 q .. 64 q + 63, so ranks follow ascending ids:
  // lane q < 16 takes word q's popcount, and an exclusive scan gives each word's first rank.
  const int32_t cq = lane < kRowsMaxK / 64 ? __popcll(rl.bits[lane]) : 0;
  const int32_t iq = dpp_scan_i32(cq);
  const int32_t n = __builtin_amdgcn_readlane(iq, kRowsMaxK / 64 - 1);
#pragma unroll
  for (int i = 0; i < kRowsPer; ++i) {
    const int q = i * kWaves + wid;  // wave-uniform
    const int32_t first = __builtin_amdgcn_readlane(iq - cq, q);
    if ((bits[i] >> lane) & 1ull) {
      const int32_t rank = first + (int32_t)__builtin_amdgcn_mbcnt_hi((uint32_t)(bits[i] >> 32),
                                                                       __builtin_amdgcn_mbcnt_lo((uint32_t)bits[i], 0u));
      rl.list[rank] = make_int2(kThreads * i + (int32_t)threadIdx.x, rr[i].z | (rr[i].w << 16));
    }
  }
  int64_t base = 0;
  int32_t fspan = 0;
#pragma unroll
  for (int w = 0; w < kWaves; ++w) {
    base += rl.before[w];
    fspan = max(fspan, rl.span[w]);
  }
  __syncthreads();
  return RowBin{rl.list, n, base, fspan, tile_ptr_out};
}

// Single 16x16 fields of up to kRowsMaxK Gaussians (rows_in_render): the render bins its own
// tile row, so no k_bin_tiles launch precedes it.  A workgroup takes eight tile pairs of one
// tile row (ceil(ceil(C / 2) / 8) workgroups a row).  Its 512 threads test the K rectangles
// (two each, loads in flight together) against the row: a ballot per 64 Gaussians gives the
// row's mask words, and each thread adds the pairs its Gaussians have in the rows above,
// w * clamp(tr - first row, 0, h).  After a barrier each thread places its row Gaussians in the
// row list at their rank (the mask words' popcounts before its word, then its lane's rank in
// the word), with their column ranges; after a second barrier each wave renders its pair from
// the list (render16x2_body<kRows>), which also gives the segment starts in closed form.
__global__ __launch_bounds__(kRowsThreads) void k_render16x2_rows(
    Problem p, const float* __restrict__ row_coords, const float* __restrict__ col_coords,
    const GaussEval* __restrict__ ev, int64_t* tile_ptr, int64_t* ids, int64_t capacity,
    float* __restrict__ delta, uint8_t* ws, const int4* __restrict__ rects) {
  __shared__ RowLds rl;
  constexpr int kWaves = kRowsThreads / 64;
  const int32_t cp = (p.C + 1) / 2;
  const int32_t G = (cp + kWaves - 1) / kWaves;  // workgroups a tile row
  const int32_t tr = (int32_t)blockIdx.x / G;
  const int32_t pc = ((int32_t)blockIdx.x - tr * G) * kWaves + wave_id();  // the wave's pair
  const RowBin rb = bin_tile_row<kRowsThreads>(p, rects, tr, rl, tile_ptr);
  if (pc >= cp) return;  // past the row's last pair (no barrier follows)
  render16x2_body<false, true>(p, row_coords, col_coords, ev, nullptr, ids, capacity, delta, ws, nullptr, nullptr,
                               tr, 2 * pc, nullptr, MergedOut{nullptr, nullptr, 1.0f}, 0u, rb);
}

// Single 16x16 fields on the mask path with heavy-tile workgroups: the first workgroups take one
// listed heavy tile each (four waves, as k_render16<true>), the rest a pair of horizontally
// adjacent tiles a wave (R x ceil(C / 2) pairs, four a workgroup, as k_render16x2), leaving a
// heavy member of the pair to its own workgroup.
__global__ __launch_bounds__(kTileThreads) __attribute__((amdgpu_waves_per_eu(8))) void k_render16x2_heavy(
    Problem p, const float* __restrict__ row_coords, const float* __restrict__ col_coords,
    const GaussEval* __restrict__ ev, const int64_t* __restrict__ tile_ptr, int64_t* ids, int64_t capacity,
    float* __restrict__ delta, uint8_t* ws, const uint32_t* __restrict__ rowmask,
    const uint32_t* __restrict__ colmask, const int32_t* __restrict__ heavy_list, int32_t xh) {
  const int64_t T = (int64_t)p.R * p.C;
  const int64_t b = blockIdx.x;
  int64_t nh = (int64_t)reinterpret_cast<const WsHeader*>(ws)->heavy;
  if (nh > xh) {
    if (b == 0 && threadIdx.x == 0) atomicOr(&reinterpret_cast<WsHeader*>(ws)->status, GF_STATUS_CAPACITY);
    nh = xh;
  }
  if (b < nh) {  // the workgroup's four waves share one listed tile
    const int64_t t = heavy_list[b];
    render16_body(p, row_coords, col_coords, ev, tile_ptr, ids, capacity, delta, ws, rowmask, colmask,
                  tile16(p, t < 0 || t >= T ? T : t), nullptr, nullptr, wave_id(), kTileThreads / 64);
    return;
  }
  const int32_t cp = (p.C + 1) / 2;
  const int64_t pi = (b - nh) * (kTileThreads / 64) + wave_id();
  if (pi >= (int64_t)p.R * cp) return;
  const int32_t tr = (int32_t)pi / cp, tc = 2 * ((int32_t)pi - tr * cp);
  const int64_t ta = (int64_t)tr * p.C + tc;
  const bool pair = tc + 1 < p.C;
  const int64_t s0 = tile_ptr[ta], s1 = tile_ptr[ta + 1], s2 = pair ? tile_ptr[ta + 2] : s1;
  // the listing rule of k_bin_tiles: a tile of more than p.heavy Gaussians is heavy
  const uint32_t skip = (s1 - s0 > p.heavy ? 1u : 0u) | (pair && s2 - s1 > p.heavy ? 2u : 0u);
  if (skip == (pair ? 3u : 1u)) return;
  render16x2_body<false>(p, row_coords, col_coords, ev, tile_ptr, ids, capacity, delta, ws, rowmask, colmask, tr,
                         tc, nullptr, MergedOut{nullptr, nullptr, 1.0f}, skip);
}

template <bool kHeavy>
__global__ __launch_bounds__(kTileThreads) void k_render16(
    Problem p, const float* __restrict__ row_coords, const float* __restrict__ col_coords,
    const GaussEval* __restrict__ ev, const int64_t* __restrict__ tile_ptr, int64_t* ids,
    int64_t capacity, float* __restrict__ delta, uint8_t* ws, const uint32_t* __restrict__ rowmask,
    const uint32_t* __restrict__ colmask, const int4* __restrict__ rects, int64_t* __restrict__ tile_ptr_out,
    const int32_t* __restrict__ heavy_list, int32_t xh) {
  HeavyItem it;
  if constexpr (kHeavy) {
    it = heavy_item(p, heavy_list, &reinterpret_cast<const WsHeader*>(ws)->heavy, xh,
                    &reinterpret_cast<WsHeader*>(ws)->status);
  } else {
    it.st = sub_tile(p, blockIdx.x, wave_id());
    it.q = 0;
    it.F = 1;
  }
  render16_body(p, row_coords, col_coords, ev, tile_ptr, ids, capacity, delta, ws, rowmask, colmask, it.st,
                rects, tile_ptr_out, it.q, it.F);
}

// Any tile shape: each thread evaluates pixels p = tid, tid+256, ... of the tile.
__global__ __launch_bounds__(kTileThreads) void k_render_any(
    Problem p, const float* __restrict__ row_coords, const float* __restrict__ col_coords,
    const GaussEval* __restrict__ ev, const int64_t* __restrict__ tile_ptr, int64_t* ids,
    int64_t capacity, float* __restrict__ delta, uint8_t* ws) {
  __shared__ int32_t keys[kSortLdsWords];
  __shared__ int64_t small_lds[kTileThreads / 64 + 1];
  __shared__ GaussEval gl[kTileThreads];
  WsHeader* hdr = reinterpret_cast<WsHeader*>(ws);
  const int32_t t = blockIdx.x;
  const int32_t tr = t / p.C, tc = t - (t / p.C) * p.C;
  int64_t s, n;
  tile_range(tile_ptr, t, capacity, &s, &n);
  int64_t* seg = ids + s;
  order_segment(seg, n, p.K, keys, small_lds, &hdr->status);
  const bool keys_in_lds = n <= kSortLdsKeys;
  const int32_t r0 = tr * p.tile_out, c0 = tc * p.tile_in;
  const int32_t r1 = min(r0 + p.tile_out, p.M), c1 = min(c0 + p.tile_in, p.N);
  const int32_t w = c1 - c0;
  const int32_t npx = (r1 - r0) * w;
  for (int32_t px0 = 0; px0 < npx; px0 += kTileThreads) {
    const int32_t px = px0 + (int32_t)threadIdx.x;
    const bool have = px < npx;
    const int32_t r = r0 + (have ? px / w : 0);
    const int32_t c = c0 + (have ? px - (px / w) * w : 0);
    const float x = row_coords[r], y = col_coords[c];
    float acc = 0.0f;
    for (int64_t j0 = 0; j0 < n; j0 += kTileThreads) {
      const int nj = (int)((n - j0) < kTileThreads ? (n - j0) : kTileThreads);
      __syncthreads();
      if ((int)threadIdx.x < nj) {
        const int64_t g = keys_in_lds ? (int64_t)keys[j0 + threadIdx.x] : seg[j0 + threadIdx.x];
        if (g >= 0 && g < p.K) {
          gl[threadIdx.x] = load_eval(ev, g);
        } else {
          gl[threadIdx.x] = zero_eval();
          set_status(&hdr->status, GF_STATUS_COUNT_MISMATCH);
        }
      }
      __syncthreads();
      for (int j = 0; j < nj; ++j) {
        const GaussEval v = gl[j];
        acc = fmaf(v.w, basis_q(p, quad_form(v, x - v.mu0, y - v.mu1)), acc);
      }
    }
    if (have) store_stream(delta + (int64_t)r * p.N + c, acc);
  }
}

// ------------------------------------------------------------------------------------------
// Backward.
//
// Six moments of one Gaussian over a set of pixels (e = basis without normalisation):
//   S0 = sum g e, S1 = sum g e dx, S2 = sum g e dy, S3 = sum g e dx^2, S4 = sum g e dx dy,
//   S5 = sum g e dy^2.
// The reference zeroes the quadratic-form terms of pixels whose form is clamped (q > clamp or
// q < 0); there e <= e^{-clamp/2} (4e-18 for clamp 80) or the pixel sits at the centre, so
// those terms are below fp32 resolution of the sums and are kept.

template <typename Idx>
__device__ inline void backward_tile_checks(const Problem& p, const Idx* __restrict__ tile_ptr,
                                            int64_t t, int64_t num_pairs, uint32_t* status,
                                            int64_t* s_out, int64_t* n_out) {
  const int64_t T = (int64_t)p.R * p.C;
  int64_t s = (int64_t)tile_ptr[t], e = (int64_t)tile_ptr[t + 1];
  if (threadIdx.x == 0) {
    if (s < 0 || e < s || e > num_pairs) set_status(status, GF_STATUS_TILE_PTR_ORDER);
    if (t == T - 1 && e != num_pairs) set_status(status, GF_STATUS_TILE_PTR_LAST);
  }
  if (s < 0) s = 0;
  if (e > num_pairs) e = num_pairs;
  *s_out = s;
  *n_out = e > s ? e - s : 0;
}

// Loads Gaussians [j0, j0+nj) of the tile into LDS; invalid ids get gid -1.
template <typename GIdx>
__device__ inline void stage_gaussians(const Problem& p, const GIdx* __restrict__ gids, int64_t s,
                                       int64_t j0, int nj, const float* __restrict__ mu,
                                       const float* __restrict__ chol_raw,
                                       const GaussEval* __restrict__ ev, GaussEval* gl,
                                       int32_t* gid_lds, uint32_t* status) {
  if ((int)threadIdx.x < nj) {
    const int64_t g = (int64_t)gids[s + j0 + threadIdx.x];
    if (g < 0 || g >= p.K) {
      set_status(status, g < 0 ? GF_STATUS_IDS_NEGATIVE : GF_STATUS_IDS_RANGE);
      gid_lds[threadIdx.x] = -1;
      gl[threadIdx.x] = zero_eval();
    } else {
      gl[threadIdx.x] = ev ? load_eval(ev, g) : eval_geom(p, mu, chol_raw, nullptr, g);
      gid_lds[threadIdx.x] = (int32_t)g;
    }
  }
}

// 16x16 tiles, one wave per tile (tile blockIdx.x * 4 + wave).  Lane l: slot = l/16, row =
// l%16; per round the four slots take four Gaussians of the tile and each lane sums its row's
// 16 pixels.  Gaussian constants are computed one per lane for up to 64 Gaussians at a time
// and fetched by slot with a lane permute.
// The moments of tile t (16x16) of one field by one wave.
// kEvalGiven: ev is never null (batches), so the per-Gaussian recomputation from mu / chol_raw
// (the exact softplus chain) is left out of the kernel, with its registers.
template <typename TpIdx, typename GIdx, bool kTransposeSums, bool kMaskClamp, bool kManyRounds = kTransposeSums,
          bool kEvalGiven = false, bool kDirect = false>
__device__ __forceinline__ void bwd16_body(
    const Problem& p, const float* __restrict__ grad, const float* __restrict__ row_coords,
    const float* __restrict__ col_coords, const float* __restrict__ mu,
    const float* __restrict__ chol_raw, const GaussEval* __restrict__ ev,
    const TpIdx* __restrict__ tile_ptr, const GIdx* __restrict__ gids, int64_t num_pairs,
    uint8_t* ws, const BwdLayout& L, const SubTile& st, int q = 0, int F = 1,
    const float4* __restrict__ dcoef = nullptr, float* __restrict__ dgrad = nullptr) {
  // kDirect (row sums only): each tile's moments go through the Gaussian's chain-rule map
  // (dcoef, store_dcoef) and the gradients are added straight into the Gaussian's slot of dgrad
  // (direct_slot), so that no finish pass follows.
  static_assert(!kDirect || !kTransposeSums, "direct gradients take the row-sum reduction");
  // F > 1 (heavy tiles): the F = 4 waves of the workgroup share tile st, wave q taking chunks
  // q, q + F, ... of kHeavyChunk Gaussians (and their indefinite-form pass).
  const int cs = F > 1 ? kHeavyChunk : 64;
  WsHeader* hdr = reinterpret_cast<WsHeader*>(ws);
  float* acc = reinterpret_cast<float*>(ws + L.acc);
  const int lane = threadIdx.x & 63;
  const int64_t T = (int64_t)p.R * p.C;
  const int64_t t = st.t;
  if (t >= T) return;
  const int32_t r0 = st.r0, c0 = st.c0;
  const int64_t stripe = st.sidx & (p.S - 1);
  float* const acc_s = acc + 8 * acc_slot(p, 0, stripe);  // Gaussian 0's slot in this tile's stripe
  const bool hb3 = (lane & 8) != 0, hb2 = (lane & 4) != 0, hb1 = (lane & 2) != 0;
  const bool atomic_lane = (lane & 1) == 0 && (lane & 15) < 12;
  const int slot = lane >> 4, row = lane & 15;
  const int32_t pr = r0 + row;
  // This lane's row of dL/d(delta) (0 outside the matrix) and the tile's coordinates are
  // requested before the segment bounds, on which they do not depend.  The wave reads the 16x16
  // block of dL/d(delta) once, a float4 per lane with the nontemporal hint (the bytes are read
  // once, and keeping them out of L2 keeps the accumulator and constant lines there), and each
  // lane takes its row from LDS (row stride 20 floats: the 16 rows' float4 reads fall in
  // distinct banks).
  // Tiles of several rounds (kManyRounds: dense fields, batches, heavy-tile kernels) without
  // the clamp mask (kShifted) take their moments about the tile's middle column y8 (below): each
  // lane also stages g (y - y8) and g (y - y8)^2 for its four columns, so that a round weights
  // one exponential with three FMAs.  The per-tile set-up is repaid over several rounds (at
  // cfg3's one round a tile it is not).  LDS row stride: 52 floats there (g, g yd, g yd^2 and
  // pad), 20 otherwise; either way the 16 rows' float4 reads fall in distinct banks.
  constexpr bool kShifted = !kMaskClamp && kManyRounds;
  constexpr int kGs = kShifted ? 52 : 20;
  __shared__ float gtile[kTileThreads / 64][16 * 52];
  float* gt = gtile[__builtin_amdgcn_readfirstlane((int32_t)(threadIdx.x >> 6))];
  float gv[16], yv[16];
  float ydl[4] = {0.f, 0.f, 0.f, 0.f};  // kShifted: the lane's four column offsets from column 8
  {
    const int32_t lr = r0 + (lane >> 2), lc = c0 + ((lane & 3) << 2);
    const float* gp = grad + (int64_t)min(lr, p.M - 1) * p.N + lc;
    float4 g4 = make_float4(0.f, 0.f, 0.f, 0.f);
    // kShifted: the tile inside the matrix, rows of N % 4 == 0 floats from a 16-byte aligned
    // base, so that every lane's float4 is aligned (the same answer in every lane: a scalar
    // branch; cfg4's backward 318 -> 305 us; the sparse-tile kernel measured 0.2 us slower with it)
    const bool inner = kShifted && c0 + 15 < p.N && (p.N & 3) == 0 &&
                       (reinterpret_cast<uintptr_t>(grad + c0) & 15) == 0;
    if (inner) {
      if (lr < p.M) g4 = load4_stream(gp);
    } else if (lr < p.M) {
      if (lc + 3 < p.N && ((reinterpret_cast<uintptr_t>(gp) & 15) == 0)) {
        g4 = load4_stream(gp);
      } else {
        g4.x = lc < p.N ? load_stream(gp) : 0.f;
        g4.y = lc + 1 < p.N ? load_stream(gp + 1) : 0.f;
        g4.z = lc + 2 < p.N ? load_stream(gp + 2) : 0.f;
        g4.w = lc + 3 < p.N ? load_stream(gp + 3) : 0.f;
      }
    }
    float* gw = gt + (lane >> 2) * kGs + ((lane & 3) << 2);
    *reinterpret_cast<float4*>(gw) = g4;
    if (kShifted) {
      // the lane's four column offsets (lanes 0..3 hold the tile's 16, the scalar yd[] below)
      const float yf = col_coords[min(c0 + 8, p.N - 1)];
#pragma unroll
      for (int i = 0; i < 4; ++i) ydl[i] = col_coords[min(lc + i, p.N - 1)] - yf;
      const float4 gy = make_float4(g4.x * ydl[0], g4.y * ydl[1], g4.z * ydl[2], g4.w * ydl[3]);
      *reinterpret_cast<float4*>(gw + 16) = gy;
      *reinterpret_cast<float4*>(gw + 32) = make_float4(gy.x * ydl[0], gy.y * ydl[1], gy.z * ydl[2], gy.w * ydl[3]);
      // the 16 column offsets, a float4 per column group in the pad of rows 0..3, for the split
      // rounds below (whose lanes take different columns)
      if (lane < 4) *reinterpret_cast<float4*>(gt + lane * kGs + 48) = make_float4(ydl[0], ydl[1], ydl[2], ydl[3]);
    }
    wave_sync();
    if (!kShifted) {
#pragma unroll
      for (int c = 0; c < 16; c += 4) {
        const float4 v = *reinterpret_cast<const float4*>(gt + row * kGs + c);
        gv[c] = v.x;
        gv[c + 1] = v.y;
        gv[c + 2] = v.z;
        gv[c + 3] = v.w;
      }
    }
  }
  // (the same 16 addresses in every lane: inside the matrix, four aligned float4 from one base)
  if (c0 + 15 < p.N && ((reinterpret_cast<uintptr_t>(col_coords + c0) & 15) == 0)) {
    const float4* yq = reinterpret_cast<const float4*>(col_coords + c0);
#pragma unroll
    for (int c = 0; c < 4; ++c) {
      const float4 v = yq[c];
      yv[4 * c] = v.x;
      yv[4 * c + 1] = v.y;
      yv[4 * c + 2] = v.z;
      yv[4 * c + 3] = v.w;
    }
  } else {
#pragma unroll
    for (int c = 0; c < 16; ++c) yv[c] = col_coords[min(c0 + c, p.N - 1)];
  }
  // kShifted: columns as offsets from the tile's middle one, column 8 (uniform: scalar
  // registers), for the moments about that column below: column c's is lane c / 4's ydl[c % 4].
  float yd[16];
#pragma unroll
  for (int c = 0; c < 16; ++c)
    yd[c] = kShifted ? __int_as_float(__builtin_amdgcn_readlane(__float_as_int(ydl[c & 3]), c >> 2)) : 0.0f;
  const float x = row_coords[min(pr, p.M - 1)];
  int64_t s = (int64_t)tile_ptr[t], e = (int64_t)tile_ptr[t + 1];
  num_pairs = live_pairs(p, num_pairs);
  const int64_t Kl = live_k(p);
  if (lane == 0) {
    if (s < 0 || e < s || e > num_pairs) set_status(&hdr->status, GF_STATUS_TILE_PTR_ORDER);
    if (t == T - 1 && e != num_pairs) set_status(&hdr->status, GF_STATUS_TILE_PTR_LAST);
  }
  if (s < 0) s = 0;
  if (e > num_pairs) e = num_pairs;
  const int64_t n = e > s ? e - s : 0;
  if (n == 0) return;
  if (F == 1 && p.heavy > 0 && n > p.heavy) return;  // a heavy-tile workgroup's

  bool tile_general = false;
  for (int64_t j0 = q * cs; j0 < n; j0 += F * cs) {
    const int nj = (int)((n - j0) < cs ? (n - j0) : cs);
    GaussEval my = zero_eval();
    int32_t myg = -1;
    if (lane < nj) {
      const int64_t g = (int64_t)gids[s + j0 + lane];
      if (g < 0 || g >= Kl) {
        set_status(&hdr->status, g < 0 ? GF_STATUS_IDS_NEGATIVE : GF_STATUS_IDS_RANGE);
      } else {
        my = (kEvalGiven || ev) ? load_eval(ev, g) : eval_geom(p, mu, chol_raw, nullptr, g);
        myg = (int32_t)g;
      }
    }
    const bool chunk_general = __builtin_amdgcn_ballot_w64(lane < nj && my.gen != 0.0f) != 0;
    // kShifted: a last round of one or two Gaussians splits their columns over the four slots
    // (two slots of eight columns each, or four of four) instead of leaving slots empty, and the
    // slots' partial moments are added before the atomics.  That round is the second pass of
    // the unrolled loop below (split is a constant in each copy), so that the full rounds carry
    // none of its work.
    const int tail = kShifted && ((nj & 3) == 1 || (nj & 3) == 2) ? (nj & 3) : 0;
#pragma unroll
    for (int pass = 0; pass < (kShifted ? 2 : 1); ++pass) {
    const bool split = pass == 1;
    for (int jb = split ? nj - tail : 0; jb < (split ? nj : nj - tail); jb += 4) {
      const int rem = nj - jb;  // wave-uniform
      const int j = split ? jb + (rem == 2 ? slot >> 1 : 0) : jb + slot;
      const int part = split ? (rem == 2 ? slot & 1 : slot) : 0;
      const int addr = j < nj ? j << 2 : 0;  // ds_bpermute byte address of the slot's lane
      auto from = [&](float v) { return __int_as_float(__builtin_amdgcn_ds_bpermute(addr, __float_as_int(v))); };
      const float mu0 = from(my.mu0), mu1 = from(my.mu1);
      const float wa = from(my.wa), wb = from(my.wb);
      const float wc = from(my.wc);
      const float gen = chunk_general ? from(my.gen) : 0.0f;
      int32_t g = __builtin_amdgcn_ds_bpermute(addr, myg);
      if (j >= nj) g = -1;
      const float dx = x - mu0;
      const float a = wa * dx;
      const float A = a * a;
      const float b = wb * dx;
      if (chunk_general && gen != 0.0f) g = -1;  // indefinite form: the pass below
      // kDirect: lanes 10..15 of a slot take output row - 10 of the slot's Gaussian; its map
      // row is requested here, before the pixel loop that hides the load
      float4 cf = make_float4(0.f, 0.f, 0.f, 0.f);
      if (kDirect && row >= 10 && g >= 0) cf = dcoef[6 * (uint32_t)g + (uint32_t)(row - 10)];
      float t0 = 0.f, t2 = 0.f, t3 = 0.f, tq = 0.f;
      if (kMaskClamp) {
#pragma unroll
        for (int c = 0; c < 16; ++c) {
          // clamped pixels (q > clamp_quad) carry no quadratic-form gradient (the reference's
          // clamp mask, backward.cu:316-320,336-338): they add to S0 only
          const float dy = yv[c] - mu1;
          const float z = fmaf(wc, dy, b);
          const float qv = -fmaf(z, z, A);
          const float ge = gv[c] * __builtin_amdgcn_exp2f(__builtin_amdgcn_fmed3f(qv, p.q_lo, 0.0f));
          t0 += ge;
          const float gq = qv < p.q_lo ? 0.0f : ge;
          tq += gq;
          const float tt = gq * dy;
          t2 += tt;
          t3 = fmaf(tt, dy, t3);
        }
      } else if (kShifted) {
        // Moments about the tile's middle column y8: with dy = yd_c + dl, dl = y8 - mu1,
        //   S(ge dy) = S(ge yd) + dl S(ge),  S(ge dy^2) = S(ge yd^2) + dl (2 S(ge yd) + dl S(ge)),
        // and z = wc dy + b = wc yd_c + z0 with z0 = wc dl + b.  The shift cancels by up to
        // (offset / width)^2, so the origin sits mid-tile (offsets of -8..7 pixels).  With clamp_quad >= 80 (or none)
        // the clamp only floors bases below e^-40 (a difference below e^-40 |g| per pixel), so
        // the floor is dropped here and below, as in the render.
        const float dl = yv[8] - mu1;
        const float z0 = fmaf(wc, dl, b);
        if (split) {
          // rem column groups (of four) per slot: groups part * rem .. part * rem + rem - 1
          for (int k = 0; k < rem; ++k) {
            const int c4 = part * rem + k;
            const float4 g4 = *reinterpret_cast<const float4*>(gt + row * kGs + 4 * c4);
            const float4 gy4 = *reinterpret_cast<const float4*>(gt + row * kGs + 16 + 4 * c4);
            const float4 gyy4 = *reinterpret_cast<const float4*>(gt + row * kGs + 32 + 4 * c4);
            const float4 yd4 = *reinterpret_cast<const float4*>(gt + c4 * kGs + 48);
            const float gq[4] = {g4.x, g4.y, g4.z, g4.w}, gyq[4] = {gy4.x, gy4.y, gy4.z, gy4.w};
            const float gyyq[4] = {gyy4.x, gyy4.y, gyy4.z, gyy4.w}, ydq[4] = {yd4.x, yd4.y, yd4.z, yd4.w};
#pragma unroll
            for (int i = 0; i < 4; ++i) {
              const float z = fmaf(wc, ydq[i], z0);
              const float e = __builtin_amdgcn_exp2f(-fmaf(z, z, A));
              t0 = fmaf(gq[i], e, t0);
              t2 = fmaf(gyq[i], e, t2);
              t3 = fmaf(gyyq[i], e, t3);
            }
          }
        } else {
#pragma unroll
        for (int c4 = 0; c4 < 4; ++c4) {
          const float4 g4 = *reinterpret_cast<const float4*>(gt + row * kGs + 4 * c4);
          const float4 gy4 = *reinterpret_cast<const float4*>(gt + row * kGs + 16 + 4 * c4);
          const float4 gyy4 = *reinterpret_cast<const float4*>(gt + row * kGs + 32 + 4 * c4);
          const float gq[4] = {g4.x, g4.y, g4.z, g4.w}, gyq[4] = {gy4.x, gy4.y, gy4.z, gy4.w};
          const float gyyq[4] = {gyy4.x, gyy4.y, gyy4.z, gyy4.w};
#pragma unroll
          for (int i = 0; i < 4; ++i) {
            const int c = 4 * c4 + i;
            const float z = c == 8 ? z0 : fmaf(wc, yd[c], z0);
            const float e = __builtin_amdgcn_exp2f(-fmaf(z, z, A));
            t0 = fmaf(gq[i], e, t0);
            t2 = fmaf(gyq[i], e, t2);
            t3 = fmaf(gyyq[i], e, t3);
          }
          // keep each group's three LDS reads beside their use (hoisted, the twelve of a round
          // would hold 48 registers)
          __builtin_amdgcn_sched_barrier(0);
        }
        }
        t3 = fmaf(dl, fmaf(dl, t0, 2.0f * t2), t3);
        t2 = fmaf(dl, t0, t2);
      } else {
#pragma unroll
        for (int c = 0; c < 16; ++c) {
          const float dy = yv[c] - mu1;
          const float z = fmaf(wc, dy, b);
          const float ge = gv[c] * __builtin_amdgcn_exp2f(-fmaf(z, z, A));
          t0 += ge;
          const float tt = ge * dy;
          t2 += tt;
          t3 = fmaf(tt, dy, t3);
        }
      }
      const float t0q = kMaskClamp ? tq : t0;  // the quadratic-form moments' share of S0
      const float m0 = t0, m1 = dx * t0q, m2 = t2, m3 = dx * dx * t0q, m4 = dx * t2, m5 = t3;
      if (kDirect) {
        // the six row sums in every lane of the row (butterfly: the same sum in each lane), then
        // lane 10 + k forms output k of the map and adds it to the Gaussian's gradient
        float s0 = dpp_row_allsum_f32(m0), s1 = dpp_row_allsum_f32(m1), s2 = dpp_row_allsum_f32(m2);
        float s3 = dpp_row_allsum_f32(m3), s4 = dpp_row_allsum_f32(m4), s5 = dpp_row_allsum_f32(m5);
        if (split) {  // (heavy tiles) the Gaussian's slots: 0 + 1 and 2 + 3 (two Gaussians) or all four
          float sv[6] = {s0, s1, s2, s3, s4, s5};
#pragma unroll
          for (int i = 0; i < 6; ++i) {
            sv[i] += __shfl_xor(sv[i], 16, 64);
            if (rem == 1) sv[i] += __shfl_xor(sv[i], 32, 64);
          }
          s0 = sv[0];
          s1 = sv[1];
          s2 = sv[2];
          s3 = sv[3];
          s4 = sv[4];
          s5 = sv[5];
        }
        const int k = row - 10;
        const float P = (k == 1 || k == 2) ? s1 : s0, Q = k < 3 ? s2 : s3;
        const float o = fmaf(cf.x, P, fmaf(cf.y, Q, fmaf(cf.z, s4, cf.w * s5)));
        if (g >= 0 && row >= 10 && part == 0) unsafeAtomicAdd(dgrad + direct_slot(g, k), o);
        continue;
      }
      if (!kTransposeSums) {
        // Six independent row sums (the shorter dependency chain, for sparse tiles where a wave
        // makes few rounds).  Lane 15 of the slot's row holds the sums; moment k moves
        // to lane 10 + k (row_shl by 5 - k) and lanes 10..15 add one each.
        const float s0 = dpp_row_sum_f32(m0), s1 = dpp_row_sum_f32(m1), s2 = dpp_row_sum_f32(m2);
        const float s3 = dpp_row_sum_f32(m3), s4 = dpp_row_sum_f32(m4), s5 = dpp_row_sum_f32(m5);
        const float v0 = dpp_f32<0x105>(s0), v1 = dpp_f32<0x104>(s1), v2 = dpp_f32<0x103>(s2);
        const float v3 = dpp_f32<0x102>(s3), v4 = dpp_f32<0x101>(s4);
        const int k = row - 10;
        if (split) {  // the Gaussian's slots: 0 + 1 and 2 + 3 (two Gaussians) or all four
          float val = k == 0 ? v0 : k == 1 ? v1 : k == 2 ? v2 : k == 3 ? v3 : k == 4 ? v4 : s5;
          val += __shfl_xor(val, 16, 64);
          if (rem == 1) val += __shfl_xor(val, 32, 64);
          if (g >= 0 && row >= 10 && part == 0)
            unsafeAtomicAdd(acc_s + (8u * (uint64_t)(uint32_t)g + (uint32_t)k), val);
        } else if (g >= 0 && row >= 10) {
          const float val = k == 0 ? v0 : k == 1 ? v1 : k == 2 ? v2 : k == 3 ? v3 : k == 4 ? v4 : s5;
          unsafeAtomicAdd(acc_s + (8u * (uint64_t)(uint32_t)g + (uint32_t)k), val);
        }
        continue;
      }
      // Dense tiles and batches (many rounds per wave): fewer instructions.  The six moments summed over the
      // slot's 16 lanes by recursive halving: each step keeps
      // half of a lane's values, sends the other half to its partner (lane ^ 15, ^ 7, ^ 2, ^ 1:
      // row_mirror, row_half_mirror, two quad_perms) and adds what it receives.  Lane r ends
      // with moment r >> 1 (moments 6, 7 are zero padding); even lanes 0..10 add it atomically.
      // Each step adds the partner's copy of both halves in every lane (one DPP add each) and
      // then, for the lanes that keep the second half, overwrites with that half's sum (a DPP
      // add under a bank mask): two instructions per kept pair instead of two selects and an
      // add.  The halves a lane drops carry whatever they carry; they only reach lanes 12..15
      // (the padding moments, no atomics).  Each sum is the same two operands as a select-and-
      // add, so the results are bit-identical (no contraction: m1 and m3 are products, which
      // an fma would fold into the first add, unrounded).
      float d;
      {
#pragma clang fp contract(off)
        const float a0 = row_mirror_sum_upper(dpp_f32<0x140>(m0) + m0, m4);
        const float a1 = row_mirror_sum_upper(dpp_f32<0x140>(m1) + m1, m5);
        const float a2 = dpp_f32<0x140>(m2) + m2;  // lanes 8..15: padding
        const float a3 = dpp_f32<0x140>(m3) + m3;
        const float c0 = row_half_mirror_sum_odd_banks(dpp_f32<0x141>(a0) + a0, a2);
        const float c1 = row_half_mirror_sum_odd_banks(dpp_f32<0x141>(a1) + a1, a3);
        d = pair_sum_all_lanes((hb1 ? c1 : c0) + dpp_f32<0x4e>(hb1 ? c0 : c1));
      }
      if (split) {  // the Gaussian's slots: 0 + 1 and 2 + 3 (two Gaussians) or all four
        d += __shfl_xor(d, 16, 64);
        if (rem == 1) d += __shfl_xor(d, 32, 64);
      }
      if (g >= 0 && atomic_lane && part == 0)
        unsafeAtomicAdd(acc_s + (8u * (uint64_t)(uint32_t)g + (uint32_t)(row >> 1)), d);
    }
    }
    tile_general = tile_general || chunk_general;
  }
  // Indefinite-form Gaussians of the tile (q' = z^2 - a^2; rare), after the rounds above so
  // that the row registers are free: lanes 0..15 take one tile row each, the pixels one at a
  // time from memory, and the clamped pixels (q < 0 or q > clamp) add nothing to the
  // quadratic-form moments.
  if (tile_general) {
    for (int64_t j0 = q * cs; j0 < n; j0 += F * cs) {
      const int nj = (int)((n - j0) < cs ? (n - j0) : cs);
      GaussEval my = zero_eval();
      int32_t myg = -1;
      if (lane < nj) {
        const int64_t g = (int64_t)gids[s + j0 + lane];
        if (g >= 0 && g < Kl) {
          my = (kEvalGiven || ev) ? load_eval(ev, g) : eval_geom(p, mu, chol_raw, nullptr, g);
          myg = (int32_t)g;
        }
      }
      uint64_t gm = __builtin_amdgcn_ballot_w64(lane < nj && my.gen != 0.0f);
      while (gm) {
        const int j = __builtin_ctzll(gm);
        gm &= gm - 1;
        const GaussEval u = readlane_eval(my, j);
        const int32_t gj = __builtin_amdgcn_readlane(myg, j);
        float mm[6] = {0.f, 0.f, 0.f, 0.f, 0.f, 0.f};
        const int32_t pr2 = r0 + lane;
        if (lane < 16 && pr2 < p.M) {
          const float dx2 = row_coords[pr2] - u.mu0;
          const float a2 = u.wa * dx2;
          const float nA2 = -(a2 * a2);
          const float b2 = u.wb * dx2;
          const float* grow2 = grad + (int64_t)pr2 * p.N;
#pragma unroll 1
          for (int c = 0; c < 16 && c0 + c < p.N; ++c) {
            const float dy = col_coords[c0 + c] - u.mu1;
            const float z = fmaf(u.wc, dy, b2);
            const float q = fmaf(z, z, nA2);
            const float qc = __builtin_amdgcn_fmed3f(q, p.q_lo, p.q_hi);
            const float ge = grow2[c0 + c] * __builtin_amdgcn_exp2f(qc);
            mm[0] += ge;
            if (qc == q) {
              mm[1] += ge * dx2;
              mm[2] += ge * dy;
              mm[3] += ge * dx2 * dx2;
              mm[4] += ge * dx2 * dy;
              mm[5] += ge * dy * dy;
            }
          }
        }
#pragma unroll
        for (int k = 0; k < 6; ++k) mm[k] = dpp_row_sum_f32(mm[k]);  // row 0: lanes 0..15
        if (lane == 15 && gj >= 0) {
          if (kDirect) {
#pragma unroll
            for (int k = 0; k < 6; ++k) {
              const float4 c = dcoef[6 * (uint32_t)gj + (uint32_t)k];
              const float P = (k == 1 || k == 2) ? mm[1] : mm[0], Q = k < 3 ? mm[2] : mm[3];
              unsafeAtomicAdd(dgrad + direct_slot(gj, k),
                              fmaf(c.x, P, fmaf(c.y, Q, fmaf(c.z, mm[4], c.w * mm[5]))));
            }
          } else {
#pragma unroll
            for (int k = 0; k < 6; ++k)
              unsafeAtomicAdd(acc + 8 * acc_slot(p, gj, stripe) + k, mm[k]);
          }
        }
      }
    }
  }
}

// Seven waves per SIMD (72 VGPRs): the rarely taken indefinite-form pass would otherwise
// raise the register count and cost the common path occupancy.
// kEvalGiven: launched with the forward's constants (ev != null); the heavy-tile kernels always
// are, since their tile list lives in the same workspace.
template <typename TpIdx, typename GIdx, bool kTransposeSums, bool kMaskClamp, bool kHeavy, bool kEvalGiven = kHeavy,
          bool kDirect = false>
__global__ __launch_bounds__(kTileThreads) __attribute__((amdgpu_waves_per_eu(7))) void k_bwd16(
    Problem p, const float* __restrict__ grad, const float* __restrict__ row_coords,
    const float* __restrict__ col_coords, const float* __restrict__ mu,
    const float* __restrict__ chol_raw, const GaussEval* __restrict__ ev,
    const TpIdx* __restrict__ tile_ptr, const GIdx* __restrict__ gids, int64_t num_pairs,
    uint8_t* ws, BwdLayout L, const int32_t* __restrict__ heavy_list,
    const uint32_t* __restrict__ heavy_count, int32_t xh, const float4* __restrict__ dcoef,
    float* __restrict__ dgrad) {
  HeavyItem it;
  if constexpr (kHeavy) {
    it = heavy_item(p, heavy_list, heavy_count, xh, &reinterpret_cast<WsHeader*>(ws)->status);
  } else {
    it.st = sub_tile(p, blockIdx.x, wave_id());
    it.q = 0;
    it.F = 1;
  }
  bwd16_body<TpIdx, GIdx, kTransposeSums, kMaskClamp, kTransposeSums || kHeavy, kEvalGiven, kDirect>(
      p, grad, row_coords, col_coords, mu, chol_raw, ev, tile_ptr, gids, num_pairs, ws, L, it.st, it.q, it.F,
      dcoef, dgrad);
}

// ------------------------------------------------------------------------------------------
// Forward and backward of a field in one pass (gf_fwd_bwd_fused), for a caller that holds
// dL/d(delta) before the forward: the reference's tile render (forward.cu:254-368) and its
// per-pair gradient pass (backward.cu:234-388) share each pixel's exponential.  After k_prep +
// k_bin_tiles (which store the Gaussians' constants, the coverage masks, tile_ptr, the
// chain-rule maps and clear the gradient slots), one wave per 16x16 tile, four a workgroup:
//   * the tile's ids are expanded from rowmask & colmask in ascending order (the canonical order
//     of the stable sort) and written to its segment of gaussian_ids_sorted, as the render does;
//   * lanes follow the backward's layout: slot = lane / 16 takes Gaussian jb + slot of a round of
//     four, row = lane % 16 evaluates its row's 16 pixels; each evaluation feeds the pixel's
//     delta-W partial (acc[c] += amp norm e) and the six moments, which go through the
//     Gaussian's map into its gradient slot (as gf_backward_direct);
//   * indefinite forms (GaussEval.gen) are left out of the rounds and taken one at a time by
//     lanes 0..15 (slot 0: one row each, their own registers), with the clamped pixels' terms
//     dropped from the quadratic-form moments;
//   * the four slots' partial rows are added in registers with gfx950's lane swaps (halves of
//     the wave, then rows of 16 lanes): lane (slot, row) ends with columns 4 slot .. 4 slot + 3 of
//     its row, summed as (slot 0 + slot 2) + (slot 1 + slot 3), and stores them (coalesced float4
//     rows, as the render).
// delta-W therefore sums each pixel's Gaussians in a different order than the render (four
// interleaved partial sums): within fp32 rounding of it, not bit-equal.
constexpr int kFusedKeys = 128;  // ids expanded per window (a tile of more takes several windows)

// Lanes 0..31 of the result: a + (a of lane + 32); lanes 32..63: (b of lane - 32) + b
// (v_permlane32_swap exchanges lanes 32..63 of its first operand with lanes 0..31 of its second).
__device__ inline float swap32_add(float a, float b) {
  const auto r = __builtin_amdgcn_permlane32_swap(__float_as_uint(a), __float_as_uint(b), false, false);
  return __uint_as_float(r[0]) + __uint_as_float(r[1]);
}
// Rows of 16 lanes: row 2i + 0 of the result: a + (a of lane + 16); row 2i + 1: (b of lane - 16) + b
// (v_permlane16_swap exchanges the odd rows of its first operand with the even rows of its second).
__device__ inline float swap16_add(float a, float b) {
  const auto r = __builtin_amdgcn_permlane16_swap(__float_as_uint(a), __float_as_uint(b), false, false);
  return __uint_as_float(r[0]) + __uint_as_float(r[1]);
}

// kRows (rows_in_render fields): a workgroup of kRowsThreads takes eight tiles of one tile row
// (ceil(C / 8) workgroups a row), bins that row first (bin_tile_row: no k_bin_tiles launch,
// k_prep stores the chain-rule maps and clears the slots) and writes its tiles' tile_ptr
// entries; each wave takes its tile's Gaussians from the row list.
template <bool kMaskClamp, bool kRows = false>
__global__ __launch_bounds__(kRows ? kRowsThreads : kTileThreads) __attribute__((amdgpu_waves_per_eu(7))) void k_fused16(
    Problem p, const float* __restrict__ grad, const float* __restrict__ row_coords,
    const float* __restrict__ col_coords, const GaussEval* __restrict__ ev, const int64_t* __restrict__ tile_ptr,
    int64_t* __restrict__ ids, int64_t capacity, float* __restrict__ delta, uint8_t* fws,
    const uint32_t* __restrict__ rowmask, const uint32_t* __restrict__ colmask, const float4* __restrict__ dcoef,
    float* __restrict__ dgrad, const int4* __restrict__ rects = nullptr, int64_t* tile_ptr_out = nullptr) {
  constexpr int kGs = 20;  // row stride (floats) of the staged dL/d(delta) tile: conflict-free float4 reads
  constexpr int kThreads = kRows ? kRowsThreads : kTileThreads, kWaves = kThreads / 64;
  __shared__ float gstage[kWaves][16 * kGs];
  __shared__ int32_t fkeys[kTileThreads / 64][kFusedKeys];  // (not used by kRows)
  // per wave: a chunk's constants, Gaussian j in [j] (mu0, mu1, wa, wb) and [64 + j] (wc, w, id, gen)
  __shared__ float4 fevals[kWaves][128];
  WsHeader* hdr = reinterpret_cast<WsHeader*>(fws);
  const int lane = threadIdx.x & 63;
  const int wid = wave_id();
  const int64_t T = (int64_t)p.R * p.C;
  int64_t t;
  int32_t r0, c0, tr, tc;
  RowBin rb{nullptr, 0, 0, 0, nullptr};
  if constexpr (kRows) {
    __shared__ RowLds rl;
    const int32_t G = (p.C + kWaves - 1) / kWaves;  // workgroups a tile row
    tr = (int32_t)blockIdx.x / G;
    tc = ((int32_t)blockIdx.x - tr * G) * kWaves + wid;
    rb = bin_tile_row<kThreads>(p, rects, tr, rl, tile_ptr_out);
    if (tc >= p.C) return;  // past the row's last tile (no barrier follows)
    t = (int64_t)tr * p.C + tc;
    r0 = tr * 16;
    c0 = tc * 16;
  } else {
    const SubTile st = sub_tile(p, blockIdx.x, wid);
    t = st.t;
    if (t >= T) return;
    r0 = st.r0;
    c0 = st.c0;
    tr = (int32_t)(t / p.C);
    tc = (int32_t)(t - (int64_t)tr * p.C);
  }
  const int slot = lane >> 4, row = lane & 15;
  float* gt = gstage[wid];
  float yv[16];
  {
    const int32_t lr = r0 + (lane >> 2), lc = c0 + ((lane & 3) << 2);
    const float* gp = grad + (int64_t)min(lr, p.M - 1) * p.N + lc;
    float4 g4 = make_float4(0.f, 0.f, 0.f, 0.f);
    if (lr < p.M) {
      if (lc + 3 < p.N && ((reinterpret_cast<uintptr_t>(gp) & 15) == 0)) {
        g4 = load4_stream(gp);
      } else {
        g4.x = lc < p.N ? load_stream(gp) : 0.f;
        g4.y = lc + 1 < p.N ? load_stream(gp + 1) : 0.f;
        g4.z = lc + 2 < p.N ? load_stream(gp + 2) : 0.f;
        g4.w = lc + 3 < p.N ? load_stream(gp + 3) : 0.f;
      }
    }
    *reinterpret_cast<float4*>(gt + (lane >> 2) * kGs + ((lane & 3) << 2)) = g4;
    wave_sync();
  }
  // The lane's row of dL/d(delta), four columns at a time from the stage (held in LDS for the
  // whole tile rather than in 16 registers: the kernel then fits seven waves per SIMD).
  const float* grow = gt + row * kGs;
  auto g4_at = [&](int c4) { return *reinterpret_cast<const float4*>(grow + 4 * c4); };
  if (c0 + 15 < p.N && ((reinterpret_cast<uintptr_t>(col_coords + c0) & 15) == 0)) {
    const float4* yq = reinterpret_cast<const float4*>(col_coords + c0);
#pragma unroll
    for (int c = 0; c < 4; ++c) {
      const float4 v = yq[c];
      yv[4 * c] = v.x;
      yv[4 * c + 1] = v.y;
      yv[4 * c + 2] = v.z;
      yv[4 * c + 3] = v.w;
    }
  } else {
#pragma unroll
    for (int c = 0; c < 16; ++c) yv[c] = col_coords[min(c0 + c, p.N - 1)];
  }
  // the tile's column coordinates are the same in every lane: scalar registers
#pragma unroll
  for (int c = 0; c < 16; ++c) yv[c] = __int_as_float(__builtin_amdgcn_readfirstlane(__float_as_int(yv[c])));
  const float x = row_coords[min(r0 + row, p.M - 1)];
  int64_t s, count;
  int32_t key0 = 0;  // kRows: the first 64 row entries' keys and constants
  bool keep0 = false;
  GaussEval pre0 = zero_eval();
  if constexpr (kRows) {
    // the tile's segment start in closed form (as render16x2_body<kRows>) and its count
    int32_t before = 0, cnt = 0;
    for (int32_t j = lane; j < rb.n; j += 64) {
      const int2 e = rb.list[j];
      const int32_t z = e.y & 0xffff, w = e.y >> 16;
      const bool in = z <= tc && tc <= w;
      before += clamp_i32(tc - z, 0, w - z + 1);
      cnt += in ? 1 : 0;
      if (j < 64) {
        keep0 = in;
        key0 = e.x;
        if (in) pre0 = load_eval(ev, e.x);
      }
    }
    s = rb.base + __builtin_amdgcn_readlane(dpp_scan_i32(before), 63);
    count = __builtin_amdgcn_readlane(dpp_scan_i32(cnt), 63);
    if (lane == 0) {
      rb.tile_ptr_out[t] = s;
      if (t == T - 1) {
        rb.tile_ptr_out[T] = s + count;
        *hdr->num_pairs = s + count;
        hdr->pairs = s + count;
        hdr->max_span = rb.span;
      }
    }
  } else {
    s = tile_ptr[t];
    count = tile_ptr[t + 1] - s;
  }
  // ids are written to [s, s + room): none for a segment below the id buffer or reversed
  const int64_t room = s < 0 ? 0 : capacity - s < count ? (capacity - s > 0 ? capacity - s : 0) : count;
  if ((s < 0 || count < 0) && lane == 0) set_status(&hdr->status, GF_STATUS_TILE_PTR_ORDER);
  float acc[16];
#pragma unroll
  for (int c = 0; c < 16; ++c) acc[c] = 0.f;

  // The rounds over a chunk of nj <= 64 Gaussians, staged in the wave's fevals (Gaussian j at
  // [j], [64 + j]); chunk_general: some of them have the indefinite form.
  float4* ew = fevals[wid];
  auto run_chunk = [&](int nj, bool chunk_general) {
    for (int jb = 0; jb < nj; jb += 4) {
      const int j = min(jb + slot, nj - 1);  // a slot past the chunk reads a real Gaussian, unused
      const float4 ea = ew[j], eb = ew[64 + j];
      const float mu0 = ea.x, mu1 = ea.y, wa = ea.z, wb = ea.w;
      const float wc = eb.x, w = eb.y, gen = eb.w;
      int32_t g = __float_as_int(eb.z);
      const bool live = jb + slot < nj && !(chunk_general && gen != 0.0f);  // indefinite forms: below
      if (!live) g = -1;
      const float wr = live ? w : 0.0f;
      const float dx = x - mu0;
      const float a = wa * dx;
      const float A = a * a;
      const float b = wb * dx;
      // lanes 10..15 of a slot take output row - 10 of the slot's Gaussian's map
      float4 cf = make_float4(0.f, 0.f, 0.f, 0.f);
      if (row >= 10 && g >= 0) cf = dcoef[6 * (uint32_t)g + (uint32_t)(row - 10)];
      float t0 = 0.f, t2 = 0.f, t3 = 0.f, tq = 0.f;
      float4 g4 = g4_at(0);
#pragma unroll
      for (int c = 0; c < 16; ++c) {
        if ((c & 3) == 0 && c > 0) g4 = g4_at(c >> 2);
        const float gc = (c & 3) == 0 ? g4.x : (c & 3) == 1 ? g4.y : (c & 3) == 2 ? g4.z : g4.w;
        const float dy = yv[c] - mu1;
        const float z = fmaf(wc, dy, b);
        if (kMaskClamp) {
          // the render's floored basis; clamped pixels (q > clamp_quad) add to S0 only (the
          // reference's clamp mask, backward.cu:316-320,336-338)
          const float qv = -fmaf(z, z, A);
          const float e = __builtin_amdgcn_exp2f(__builtin_amdgcn_fmed3f(qv, p.q_lo, 0.0f));
          acc[c] = fmaf(wr, e, acc[c]);
          const float ge = gc * e;
          t0 += ge;
          const float gq = qv < p.q_lo ? 0.0f : ge;
          tq += gq;
          const float tt = gq * dy;
          t2 += tt;
          t3 = fmaf(tt, dy, t3);
        } else {
          // clamp >= 80 (or none): the floor only moves bases below e^-40, dropped as in the
          // render and the backward
          const float e = __builtin_amdgcn_exp2f(-fmaf(z, z, A));
          acc[c] = fmaf(wr, e, acc[c]);
          const float ge = gc * e;
          t0 += ge;
          const float tt = ge * dy;
          t2 += tt;
          t3 = fmaf(tt, dy, t3);
        }
        // keep each group of four columns' work beside its LDS read (interleaved across groups,
        // the round would hold more registers than seven waves a SIMD leave)
        if ((c & 3) == 3) __builtin_amdgcn_sched_barrier(0);
      }
      const float t0q = kMaskClamp ? tq : t0;
      const float m0 = t0, m1 = dx * t0q, m2 = t2, m3 = dx * dx * t0q, m4 = dx * t2, m5 = t3;
      const float s0 = dpp_row_allsum_f32(m0), s1 = dpp_row_allsum_f32(m1), s2 = dpp_row_allsum_f32(m2);
      const float s3 = dpp_row_allsum_f32(m3), s4 = dpp_row_allsum_f32(m4), s5 = dpp_row_allsum_f32(m5);
      const int k = row - 10;
      const float P = (k == 1 || k == 2) ? s1 : s0, Q = k < 3 ? s2 : s3;
      const float o = fmaf(cf.x, P, fmaf(cf.y, Q, fmaf(cf.z, s4, cf.w * s5)));
      if (g >= 0 && row >= 10) unsafeAtomicAdd(dgrad + direct_slot(g, k), o);
    }
    if (chunk_general) {
      // indefinite forms of the chunk (q' = z^2 - a^2; rare), one at a time: lanes 0..15 (slot 0)
      // hold rows 0..15 of the tile in their own registers (x, gv, acc)
      uint64_t gm = __builtin_amdgcn_ballot_w64(lane < nj && ew[64 + min(lane, nj - 1)].w != 0.0f);
      while (gm) {
        const int j = __builtin_ctzll(gm);
        gm &= gm - 1;
        const float4 ea = ew[j], eb = ew[64 + j];
        GaussEval u;
        u.mu0 = ea.x;
        u.mu1 = ea.y;
        u.wa = ea.z;
        u.wb = ea.w;
        u.wc = eb.x;
        u.w = eb.y;
        const int32_t gj = __float_as_int(eb.z);
        float mm[6] = {0.f, 0.f, 0.f, 0.f, 0.f, 0.f};
        if (lane < 16) {
          const float dx2 = x - u.mu0;
          const float a2 = u.wa * dx2;
          const float nA2 = -(a2 * a2);
          const float b2 = u.wb * dx2;
#pragma unroll
          for (int c = 0; c < 16; ++c) {
            const float4 gq4 = g4_at(c >> 2);
            const float gc = (c & 3) == 0 ? gq4.x : (c & 3) == 1 ? gq4.y : (c & 3) == 2 ? gq4.z : gq4.w;
            const float dy = yv[c] - u.mu1;
            const float z = fmaf(u.wc, dy, b2);
            const float q = fmaf(z, z, nA2);
            const float qc = __builtin_amdgcn_fmed3f(q, p.q_lo, p.q_hi);
            const float e = __builtin_amdgcn_exp2f(qc);
            acc[c] = fmaf(u.w, e, acc[c]);
            const float ge = gc * e;
            mm[0] += ge;
            if (qc == q) {
              mm[1] += ge * dx2;
              mm[2] += ge * dy;
              mm[3] += ge * dx2 * dx2;
              mm[4] += ge * dx2 * dy;
              mm[5] += ge * dy * dy;
            }
          }
        }
#pragma unroll
        for (int kk = 0; kk < 6; ++kk) mm[kk] = dpp_row_sum_f32(mm[kk]);  // row 0: lanes 0..15
        if (lane == 15 && gj >= 0) {
#pragma unroll
          for (int kk = 0; kk < 6; ++kk) {
            const float4 c = dcoef[6 * (uint32_t)gj + (uint32_t)kk];
            const float P = (kk == 1 || kk == 2) ? mm[1] : mm[0], Q = kk < 3 ? mm[2] : mm[3];
            unsafeAtomicAdd(dgrad + direct_slot(gj, kk), fmaf(c.x, P, fmaf(c.y, Q, fmaf(c.z, mm[4], c.w * mm[5]))));
          }
        }
      }
    }
  };

  int64_t done = 0;
  if constexpr (kRows) {
    // 64 row entries at a time: the tile's Gaussians among them are a chunk, in id order
    for (int32_t j0 = 0; j0 < rb.n; j0 += 64) {
      int32_t g = key0;
      bool in = keep0;
      GaussEval my = pre0;
      if (j0 > 0) {
        in = false;
        if (j0 + lane < rb.n) {
          const int2 e = rb.list[j0 + lane];
          const int32_t z = e.y & 0xffff, w = e.y >> 16;
          in = z <= tc && tc <= w;
          g = e.x;
          if (in) my = load_eval(ev, g);
        }
      }
      const uint64_t bal = __builtin_amdgcn_ballot_w64(in);
      if (bal == 0ull) continue;  // wave-uniform
      const int nj = __popcll(bal);
      if (in) {
        const int r = (int)__builtin_amdgcn_mbcnt_hi((uint32_t)(bal >> 32), __builtin_amdgcn_mbcnt_lo((uint32_t)bal, 0u));
        if (done + r < room) ids[s + done + r] = g;
        ew[r] = make_float4(my.mu0, my.mu1, my.wa, my.wb);
        ew[64 + r] = make_float4(my.wc, my.w, __int_as_float(g), my.gen);
      }
      const bool chunk_general = __builtin_amdgcn_ballot_w64(in && my.gen != 0.0f) != 0;
      wave_sync();
      run_chunk(nj, chunk_general);
      wave_sync();  // every lane has read the chunk before the next one is staged
      done += nj;
    }
  }
  const uint32_t* rm = kRows ? nullptr : rowmask + (int64_t)tr * p.W;
  const uint32_t* cm = kRows ? nullptr : colmask + (int64_t)tc * p.W;
  int32_t* keys = fkeys[kRows ? 0 : wid];
  for (int32_t w0 = 0; !kRows && w0 < p.W; w0 += 64) {
    const int32_t w = w0 + lane;
    const uint32_t m = w < p.W ? (rm[w] & cm[w]) : 0u;
    const int32_t cnt = __popc(m);
    const int32_t inc = dpp_scan_i32(cnt);
    const int32_t tot = __builtin_amdgcn_readlane(inc, 63);
    // Expand the set bits in order, kFusedKeys positions at a time.
    for (int32_t base = 0; base < tot; base += kFusedKeys) {
      uint32_t mm = m;
      int32_t pos = inc - cnt;
      while (mm != 0u && pos < base + kFusedKeys) {
        const int32_t bit = __builtin_ctz(mm);
        mm &= mm - 1u;
        if (pos >= base) keys[pos - base] = (w << 5) + bit;
        ++pos;
      }
      wave_sync();
      const int32_t nwin = min(kFusedKeys, tot - base);
      for (int32_t j = lane; j < nwin; j += 64) {
        const int64_t sl = done + j;
        if (sl < room) ids[s + sl] = keys[j];
      }
      for (int32_t j0 = 0; j0 < nwin; j0 += 64) {
        const int nj = min(64, nwin - j0);
        bool gen_here = false;
        if (lane < nj) {
          const int32_t g = keys[j0 + lane];
          const GaussEval my = load_eval(ev, g);
          ew[lane] = make_float4(my.mu0, my.mu1, my.wa, my.wb);
          ew[64 + lane] = make_float4(my.wc, my.w, __int_as_float(g), my.gen);
          gen_here = my.gen != 0.0f;
        }
        const bool chunk_general = __builtin_amdgcn_ballot_w64(gen_here) != 0;
        wave_sync();
        run_chunk(nj, chunk_general);
        wave_sync();  // every lane has read the chunk before the next one is staged
      }
      done += nwin;
      wave_sync();  // the keys are read before the next window rewrites them
    }
  }
  if (lane == 0) {
    if (done != count) set_status(&hdr->status, GF_STATUS_COUNT_MISMATCH);
    if (room < count) set_status(&hdr->status, GF_STATUS_CAPACITY);
  }
  // The slots' partial rows summed in registers.  After the 32-lane swaps, lanes of slots 0, 1
  // hold columns 0..7 summed over slots (s, s + 2) and lanes of slots 2, 3 columns 8..15 over
  // (s - 2, s); after the 16-lane swaps, lane (slot, row) holds columns 4 slot .. 4 slot + 3 of its
  // row over all four slots.
  float h8[8];
#pragma unroll
  for (int c = 0; c < 8; ++c) h8[c] = swap32_add(acc[c], acc[c + 8]);
  float out[4];
#pragma unroll
  for (int c = 0; c < 4; ++c) out[c] = swap16_add(h8[c], h8[c + 4]);
  const int32_t opr = r0 + row, opc = c0 + (slot << 2);
  if (opr < p.M) store_row4(p, delta, MergedOut{nullptr, nullptr, 1.0f}, opr, opc, out);
}

__device__ inline float wave_sum(float v) {
#pragma unroll
  for (int o = 32; o > 0; o >>= 1) v += __shfl_xor(v, o, 64);
  return v;
}

// Any tile shape: per Gaussian, every thread sums its pixels, then a workgroup reduction.
template <typename TpIdx, typename GIdx>
__global__ __launch_bounds__(kTileThreads) void k_bwd_any(
    Problem p, const float* __restrict__ grad, const float* __restrict__ row_coords,
    const float* __restrict__ col_coords, const float* __restrict__ mu,
    const float* __restrict__ chol_raw, const GaussEval* __restrict__ ev,
    const TpIdx* __restrict__ tile_ptr, const GIdx* __restrict__ gids, int64_t num_pairs,
    uint8_t* ws, BwdLayout L) {
  __shared__ GaussEval gl[kTileThreads];
  __shared__ int32_t gid_lds[kTileThreads];
  __shared__ float red[kTileThreads / 64][8];
  WsHeader* hdr = reinterpret_cast<WsHeader*>(ws);
  float* acc = reinterpret_cast<float*>(ws + L.acc);
  const int64_t t = blockIdx.x;
  int64_t s, n;
  backward_tile_checks<TpIdx>(p, tile_ptr, t, num_pairs, &hdr->status, &s, &n);
  if (n == 0) return;
  const int lane = threadIdx.x & 63, wid = threadIdx.x >> 6;
  const int32_t tr = (int32_t)(t / p.C), tc = (int32_t)(t - (t / p.C) * p.C);
  const int32_t r0 = tr * p.tile_out, c0 = tc * p.tile_in;
  const int32_t r1 = min(r0 + p.tile_out, p.M), c1 = min(c0 + p.tile_in, p.N);
  const int32_t w = c1 - c0;
  const int32_t npx = (r1 - r0) * w;
  for (int64_t j0 = 0; j0 < n; j0 += kTileThreads) {
    const int nj = (int)((n - j0) < kTileThreads ? (n - j0) : kTileThreads);
    __syncthreads();
    stage_gaussians<GIdx>(p, gids, s, j0, nj, mu, chol_raw, ev, gl, gid_lds, &hdr->status);
    __syncthreads();
    for (int j = 0; j < nj; ++j) {
      const int32_t g = gid_lds[j];
      if (g < 0) continue;
      const GaussEval v = gl[j];
      float m[6] = {0.f, 0.f, 0.f, 0.f, 0.f, 0.f};
      for (int32_t px = threadIdx.x; px < npx; px += kTileThreads) {
        const int32_t r = r0 + px / w, c = c0 + (px - (px / w) * w);
        const float gr = grad[(int64_t)r * p.N + c];
        const float dx = row_coords[r] - v.mu0, dy = col_coords[c] - v.mu1;
        const float q = quad_form(v, dx, dy);
        const float ge = gr * basis_q(p, q);
        m[0] += ge;
        // clamped pixels carry no quadratic-form gradient (backward.cu:316-320,336-338)
        const float gq = !(q >= p.q_lo && q <= p.q_hi) ? 0.f : ge;
        m[1] += gq * dx;
        m[2] += gq * dy;
        m[3] += gq * dx * dx;
        m[4] += gq * dx * dy;
        m[5] += gq * dy * dy;
      }
#pragma unroll
      for (int k = 0; k < 6; ++k) m[k] = wave_sum(m[k]);
      if (lane == 0) {
#pragma unroll
        for (int k = 0; k < 6; ++k) red[wid][k] = m[k];
      }
      __syncthreads();
      if (threadIdx.x < 6) {
        float tot = 0.f;
#pragma unroll
        for (int q = 0; q < kTileThreads / 64; ++q) tot += red[q][threadIdx.x];
        unsafeAtomicAdd(acc + 8 * acc_slot(p, g, t & (p.S - 1)) + threadIdx.x, tot);
      }
      __syncthreads();
    }
  }
}

// Chain rule from the six moments of Gaussian g to (d_mu, d_chol_raw, d_amp), in double:
//   d_amp = norm S0;  d_mu = amp norm A (S1, S2);  dL/dA = -amp norm / 2 [[S3,S4],[S4,S5]];
//   dL/ddet = amp S0 (-norm / (2 det)) if normalize and sqrt(det) >= eps (else 0);
//   G = dL/dcov = -A (dL/dA) A + dL/ddet det A;  dL/dL = (G + G^T) L;  softplus' on the diagonal.
// A is the inverse of the fp32 covariance; the algebra follows torch's autograd of the
// reference CPU path (linalg.inv, linalg.det, L L^T, softplus).
// The chain rule for the Gaussians of one field, S = p.S threads per Gaussian: thread idx
// takes stripe idx % S of Gaussian idx / S (loads it and clears it), the S threads (adjacent
// lanes of one wave) sum the six moments with xor shuffles, and the first applies the chain
// rule.  Every lane of the wave must call it (the shuffles).
// ostride: floats between consecutive Gaussians' outputs in each of d_mu, d_chol_raw, d_amp (0:
// the arrays [K][2], [K][3], [K][1], written; 8: one slot of 8 floats per Gaussian, as
// gf_backward_direct's, added to: the one-launch kernel adds into those slots too, so both paths
// accumulate until the next forward clears them).
__device__ __forceinline__ void finish_body(
    const Problem& p, const float* __restrict__ chol_raw, const float* __restrict__ amp,
    float* __restrict__ d_mu, float* __restrict__ d_chol_raw, float* __restrict__ d_amp, uint8_t* ws,
    const BwdLayout& L, int64_t idx, const float* __restrict__ mu = nullptr,
    const float4* __restrict__ fwd_cov = nullptr, const float2* __restrict__ fwd_lfac = nullptr,
    int32_t ostride = 0, float gscale = 1.0f) {
  float* acc = reinterpret_cast<float*>(ws + L.acc);
  const int64_t g = idx / p.S;
  const int32_t st = (int32_t)(idx & (p.S - 1));
  float m[6] = {0.f, 0.f, 0.f, 0.f, 0.f, 0.f};
  const int64_t Kl = live_k(p);
  if (g < Kl) {
    float4* ag = reinterpret_cast<float4*>(acc) + 2 * acc_slot(p, g, st);
    const float4 b0 = ag[0], b1 = ag[1];
    ag[0] = make_float4(0.f, 0.f, 0.f, 0.f);
    ag[1] = make_float4(0.f, 0.f, 0.f, 0.f);
    m[0] = b0.x;
    m[1] = b0.y;
    m[2] = b0.z;
    m[3] = b0.w;
    m[4] = b1.x;
    m[5] = b1.y;
  }
  for (int32_t o = 1; o < p.S; o <<= 1) {
#pragma unroll
    for (int k = 0; k < 6; ++k) m[k] += __shfl_xor(m[k], o, 64);
  }
  if (g >= Kl || st != 0) return;
  const float raw11 = chol_raw[3 * g + 0], raw21 = chol_raw[3 * g + 1], raw22 = chol_raw[3 * g + 2];
  GfChol Lc;
  GfCov cov;
  if (fwd_cov) {  // the forward's factor and covariance (the same functions of chol_raw)
    const float2 lf = fwd_lfac[g];
    const float4 c4 = fwd_cov[g];
    Lc.l11 = lf.x;
    Lc.l21 = raw21;
    Lc.l22 = lf.y;
    cov.s00 = c4.x;
    cov.s01 = c4.y;
    cov.s11 = c4.z;
  } else {
    Lc = gf_activate_cholesky(raw11, raw21, raw22);
    cov = gf_cov_from_chol(Lc);
  }
  const GfRenderGeom rg = gf_render_geom(cov, p.normalize);
  // gscale: dL/d(delta) = gscale * the gradient the moments were taken of (a merged layer's
  // dL/d(merged weight)); the moments are linear in it
  const double gs = gscale;
  const double S0 = gs * m[0], S1 = gs * m[1], S2 = gs * m[2], S3 = gs * m[3], S4 = gs * m[4], S5 = gs * m[5];
  const double a = (double)amp[g];
  const double nrm = (double)rg.norm;
  const double an = a * nrm;
  const int64_t om = ostride ? ostride * g : 2 * g, oc = ostride ? ostride * g : 3 * g, oa = ostride ? ostride * g : g;
  // gf_backward_direct's slots accumulate (one thread per Gaussian: no other writer here)
  auto put = [ostride](float* __restrict__ out, int64_t i, float v) {
    if (ostride) out[i] += v;
    else out[i] = v;
  };
  put(d_amp, oa, (float)(nrm * S0));
  float dm0 = (float)(an * (rg.i00 * S1 + rg.i01 * S2));
  float dm1 = (float)(an * (rg.i01 * S1 + rg.i11 * S2));
  if (p.mu_tanh) {  // dL/d(mu_raw) = dL/d(mu) * (1 - tanh(mu_raw)^2), as torch's tanh backward
    const float y0 = tanhf(mu[2 * g + 0]), y1 = tanhf(mu[2 * g + 1]);
    dm0 = dm0 * (1.0f - y0 * y0);
    dm1 = dm1 * (1.0f - y1 * y1);
  }
  put(d_mu, om + 0, dm0);
  put(d_mu, om + 1, dm1);
  const double G00 = -0.5 * an * S3, G01 = -0.5 * an * S4, G11 = -0.5 * an * S5;
  const double ag00 = rg.i00 * G00 + rg.i01 * G01, ag01 = rg.i00 * G01 + rg.i01 * G11;
  const double ag10 = rg.i01 * G00 + rg.i11 * G01, ag11 = rg.i01 * G01 + rg.i11 * G11;
  double c00 = -(ag00 * rg.i00 + ag01 * rg.i01);
  double c01 = -(ag00 * rg.i01 + ag01 * rg.i11);
  double c10 = -(ag10 * rg.i00 + ag11 * rg.i01);
  double c11 = -(ag10 * rg.i01 + ag11 * rg.i11);
  if (p.normalize) {
    const float sq = gf_sqrt_rn(rg.det_f);
    if (sq >= GF_FLT_EPS) {
      const double f = a * S0 * (-nrm / 2.0);  // dL/ddet * det
      c00 += f * rg.i00;
      c01 += f * rg.i01;
      c10 += f * rg.i01;
      c11 += f * rg.i11;
    }
  }
  const double l11 = Lc.l11, l21 = Lc.l21, l22 = Lc.l22;
  const double dl11 = 2.0 * c00 * l11 + (c01 + c10) * l21;
  const double dl21 = (c10 + c01) * l11 + 2.0 * c11 * l21;
  const double dl22 = 2.0 * c11 * l22;
  put(d_chol_raw, oc + 0, (float)(dl11 * softplus_grad_f32(raw11)));
  put(d_chol_raw, oc + 1, (float)dl21);
  put(d_chol_raw, oc + 2, (float)(dl22 * softplus_grad_f32(raw22)));
}

__global__ __launch_bounds__(kTileThreads) void k_bwd_finish(
    Problem p, const float* __restrict__ chol_raw, const float* __restrict__ amp,
    float* __restrict__ d_mu, float* __restrict__ d_chol_raw, float* __restrict__ d_amp, uint8_t* ws,
    BwdLayout L, const float4* __restrict__ fwd_cov, const float2* __restrict__ fwd_lfac, int32_t ostride) {
  finish_body(p, chol_raw, amp, d_mu, d_chol_raw, d_amp, ws, L,
              (int64_t)blockIdx.x * blockDim.x + threadIdx.x, nullptr, fwd_cov, fwd_lfac, ostride);
}

// Self-test: order-independent checksum of gf_softplus_torch_cpu over all 2^32 inputs.
__device__ inline uint64_t mix64(uint64_t z) {
  z += 0x9e3779b97f4a7c15ull;
  z = (z ^ (z >> 30)) * 0xbf58476d1ce4e5b9ull;
  z = (z ^ (z >> 27)) * 0x94d049bb133111ebull;
  return z ^ (z >> 31);
}

__global__ __launch_bounds__(256) void k_selftest_softplus(unsigned long long* out) {
  uint64_t h = 0;
  const uint64_t stride = (uint64_t)gridDim.x * blockDim.x;
  for (uint64_t u = (uint64_t)blockIdx.x * blockDim.x + threadIdx.x; u < 0x100000000ull; u += stride) {
    const float y = gf_softplus_torch_cpu(gf_f32_bits((uint32_t)u));
    const uint32_t yb = (y != y) ? 0x7fc00000u : gf_bits_f32(y);
    h += mix64((u << 32) | yb);
  }
#pragma unroll
  for (int o = 32; o > 0; o >>= 1) h += __shfl_xor(h, o, 64);
  if ((threadIdx.x & 63) == 0) atomicAdd(out, (unsigned long long)h);
}

// ------------------------------------------------------------------------------------------
// Host helpers.

// Accumulator stripes of the backward: tile grids large enough to hold Gaussians that touch
// thousands of tiles (whose atomics on one cache line serialise) get 4, 8 or 32 stripes; the
// finish then reads and clears K * S * 32 bytes (one thread per stripe).  One Gaussian over the
// whole grid took cfg3's reduction from 9 to 85 us with one stripe and 24 us with 4; at 8,960
// tiles 33 us with 4 stripes and 19 us with 8.  Where the memory channels put a Gaussian's
// stripe lines depends on the accumulators' base address: above 16,384 tiles 16 stripes left
// cfg5's reduction at 37-56 us over placements, 32 at 35-39 us (64: the finish cost more than it
// saved).  Without hot Gaussians the stripes cost the finish 0.5-1.9 us.
int32_t backward_stripes(int64_t K, int64_t T) {
  (void)K;
  return T >= 16384 ? 32 : (T >= 8192 ? 8 : (T >= 2048 ? 4 : 1));
}

int make_problem(const gf_field_config* cfg, int64_t M, int64_t N, int64_t K, Problem* p) {
  if (!cfg) return set_err(GF_E_INVALID_ARGUMENT, "config must not be NULL");
  if (cfg->tile_out <= 0) return set_err(GF_E_INVALID_ARGUMENT, "tile_out must be positive");
  if (cfg->tile_in <= 0) return set_err(GF_E_INVALID_ARGUMENT, "tile_in must be positive");
  if (!(cfg->sigma_multiplier > 0.0))
    return set_err(GF_E_INVALID_ARGUMENT, "sigma_multiplier must be positive");
  if (M <= 0 || N <= 0)
    return set_err(GF_E_INVALID_ARGUMENT, "out_features and in_features must be positive");
  if (K < 0) return set_err(GF_E_INVALID_ARGUMENT, "K must be non-negative");
  if (K > INT32_MAX || M > INT32_MAX || N > INT32_MAX)
    return set_err(GF_E_INVALID_ARGUMENT, "K, out_features and in_features must be < 2^31");
  const int64_t R = (M + cfg->tile_out - 1) / cfg->tile_out, C = (N + cfg->tile_in - 1) / cfg->tile_in;
  if (R * C > INT32_MAX) return set_err(GF_E_INVALID_ARGUMENT, "too many tiles (>= 2^31)");
  p->K = K;
  p->M = (int32_t)M;
  p->N = (int32_t)N;
  // A tile larger than the matrix covers it once; clamping keeps the 32-bit tile arithmetic exact.
  p->tile_out = (int32_t)std::min<int64_t>(cfg->tile_out, M);
  p->tile_in = (int32_t)std::min<int64_t>(cfg->tile_in, N);
  p->R = (int32_t)R;
  p->C = (int32_t)C;
  p->sigma = (float)cfg->sigma_multiplier;
  if (cfg->has_clamp_quad) {
    // q in [0, clamp] -> q * kHalfLog2e in [clamp * kHalfLog2e, 0]
    p->q_lo = (float)(cfg->clamp_quad * (double)kHalfLog2e);
    p->q_hi = 0.0f;
    if (p->q_lo > p->q_hi) p->q_lo = p->q_hi;  // negative clamp: the form is pinned at 0
  } else {
    p->q_lo = -INFINITY;
    p->q_hi = INFINITY;
  }
  p->normalize = cfg->normalize ? 1 : 0;
  p->S = backward_stripes(K, R * C);
  p->mu_tanh = 0;
  p->mask_clamp = (cfg->has_clamp_quad && cfg->clamp_quad < 80.0) ? 1 : 0;
  p->heavy = 0;  // set per launch (heavy_threshold)
  p->kdev = nullptr;
  p->pdev = nullptr;
  // Mask path (no emission kernel): 16x16 or 32x32 tiles, 1 <= K <= kMaskMaxK, a tile grid
  // k_bin bins in LDS, and masks of a bounded total size.
  p->W = 0;
  if (((p->tile_out == 16 && p->tile_in == 16) || (p->tile_out == 32 && p->tile_in == 32)) && K >= 1 &&
      K <= kMaskMaxK && bin_counts_in_lds(C, K)) {
    const int64_t W = (K + 31) / 32;
    if ((R + C) * W <= kMaskMaxWords) p->W = (int32_t)W;
  }
  return GF_OK;
}

// The 16x16-block tile kernels (k_render16 / k_bwd16 and their batched forms) run 16x16
// tiles, and 32x32 tiles as four 16x16 quadrants; the render only on the mask path for 32x32
// (its emission path sorts each tile's ids in place, which four waves cannot share).
bool quad_tiles(const Problem& p) {
  return (p.tile_out == 16 && p.tile_in == 16) || (p.tile_out == 32 && p.tile_in == 32);
}
bool quad_render(const Problem& p) { return quad_tiles(p) && (p.tile_out == 16 || p.W > 0); }

// Fields with few Gaussians bin their tiles in the render, which saves the k_bin_tiles launch
// (about 4 us): each wave reads the K rectangles for its own tile's mask words and segment
// start, K/64 dependent rounds of loads.  Measured over SD1.5 shapes (320..1280 square and
// 320x768), this gains 0.4-2.3 us for K <= 256 and loses 3 us or more at K = 1024.
constexpr int64_t kTilesInRenderMaxK = 256;
constexpr int64_t kTilesInRenderMaxTests = int64_t(1) << 23;
bool tiles_in_render(const Problem& p) {
  return p.W > 0 && quad_render(p) && p.K <= kTilesInRenderMaxK &&
         (int64_t)p.R * p.C * p.K <= kTilesInRenderMaxTests;
}

// The limits of the row binning (bin_tile_row): single 16x16 fields on the mask path of at most
// kRowsMaxK Gaussians; column ranges travel as 16-bit halves, and the pair counts it sums (at
// most K * T) fit 31 bits.
bool rows_fit(const Problem& p) {
  return p.W > 0 && p.tile_out == 16 && p.tile_in == 16 && p.K <= kRowsMaxK && p.C <= 0x7fff &&
         (int64_t)p.R * p.C * p.K < (int64_t(1) << 31);
}

// Single 16x16 fields of more Gaussians, up to kRowsMaxK, bin in the pair render a tile row per
// workgroup (k_render16x2_rows): K rectangle tests per workgroup, shared by its sixteen tiles,
// instead of the k_bin_tiles launch.  (Up to 256 the per-tile form above renders faster: cfg2
// 14.05 against 14.17 us per step.)
bool rows_in_render(const Problem& p) { return rows_fit(p) && !tiles_in_render(p); }

// Either form: no k_bin_tiles launch (k_prep stores the chain-rule maps) and no heavy-tile list.
bool binned_in_render(const Problem& p) { return tiles_in_render(p) || rows_in_render(p); }

// Heavy tiles.  One wave per tile leaves a tile of many Gaussians as the tail of the render
// and the backward: at cfg5 (clustered, up to 166 Gaussians per tile) the 364 tiles of more
// than 64 Gaussians, 12% of the pairs, cost the render 12 us of 42 and the backward 19 us of
// 67.  Single 16x16 fields on the k_bin_tiles path therefore list the tiles of more than
// kHeavyTile Gaussians while binning; the render and backward give each listed tile a
// workgroup of four waves, dispatched before the one-wave-per-tile workgroups, which skip them
// (heavy_item).  With the pair render for the light tiles, thresholds 12..64 measured as cfg5 /
// cfg5c steps: 12: 100.4 / 52.6 us, 16: 85.7 / 52.7, 20: 82.3 / 53.9, 24: 80.6 / 53.7,
// 32: 81.1 / 55.3, 48: 83.7 / 58.6, 64: 87.6 / 63.6.  K <= kHeavyTile cannot make a heavy tile.
constexpr int32_t kHeavyTile = 24;
int32_t heavy_threshold(const Problem& p) {
  return p.W > 0 && p.tile_out == 16 && p.tile_in == 16 && !binned_in_render(p) && p.K > kHeavyTile
             ? kHeavyTile : 0;
}
// The kernels with heavy-tile workgroups (kHeavy) run about 1 us slower than the plain ones
// at cfg3, which has no heavy tile: the four-wave path changes the code of the one-wave path.
// They are launched for fields of many Gaussians (K >= 2048, where densification has
// clustered them) or many pairs per tile (>= 8 on average); cfg5c, clustered at 2 pairs per
// tile, has 271 heavy tiles.  Return: their extra workgroups (0: the plain kernels).  At most
// min(T, pairs / (kHeavyTile + 1)) tiles are heavy, for pairs <= pair_bound (the id
// capacity, or P); the workgroups not needed return at the end of the grid.
constexpr int64_t kHeavyMinK = 2048;
constexpr int64_t kHeavyMinPairsPerTile = 8;
int32_t heavy_grid(const Problem& p, int64_t pair_bound) {
  const int64_t T = (int64_t)p.R * p.C;
  if (heavy_threshold(p) <= 0 || pair_bound <= 0) return 0;
  if (p.K < kHeavyMinK && pair_bound < kHeavyMinPairsPerTile * T) return 0;
  const int64_t n = pair_bound / (kHeavyTile + 1);
  return (int32_t)(n < T ? n : T);
}

// Workgroups of the 16x16-block tile kernels: four 16x16 tiles or one 32x32 tile each.
int64_t quad_grid(const Problem& p) {
  const int64_t T = (int64_t)p.R * p.C;
  return p.tile_out == 32 ? T : (T + kTileThreads / 64 - 1) / (kTileThreads / 64);
}


// ------------------------------------------------------------------------------------------
// Batched fields (one launch per phase for many layers).  The plan buffer holds a header,
// one BatchLayer per field and, per kernel shape, a block -> field map:
//   tile map    4 tiles per block (backward reduce; render of the layers without tile pairs)
//   emit map    4 Gaussians per block
//   finish map  256 Gaussians per block
//   render map  4 pairs of 16x16 tiles per block (layers rendered by tile pairs)
// Each field's blocks are contiguous, so block b of a kernel handles local index
// (b - first block of its field) * per_block + wave / thread.

struct BatchLayer {
  Problem p;
  FwdLayout fl;
  BwdLayout bl;
  const float* row_coords;
  const float* col_coords;
  const float* mu;
  const float* chol_raw;
  const float* amp;
  float* delta;
  int64_t* tile_ptr;
  int64_t* num_pairs;
  int64_t* ids;
  int64_t capacity;
  uint8_t* fws;
  uint8_t* bws;
  float* d_mu;
  float* d_chol_raw;
  float* d_amp;
  int64_t tile_block0, emit_block0, finish_block0, render_block0;
  int32_t pair_render;  // rendered by tile pairs (render map); else tile by tile (tile map)
  float grad_scale;     // the backward's moments are multiplied by it (merged layers: delta_scale)
  MergedOut mo;         // merged consumer (mo.merged NULL: none)
};

// Plan regions after the header: layers, the tile / emission / finish block maps, the
// dL/d(delta) pointer of every layer (rewritten by gf_batch_set_grads) and a read-back area
// (per layer: status bits, pair count).
struct BatchHeader {
  int64_t n;
  int64_t tile_blocks, emit_blocks, finish_blocks, render_blocks;
  int64_t layers_off, tile_map_off, emit_map_off, finish_map_off, render_map_off, grad_table_off, readback_off,
      total;
};

struct BatchReadback {
  uint32_t status;
  uint32_t pad;
  int64_t pairs;
  double delta_sumsq;  // sum of delta-W^2 of the last forward
  double pad2;
};

BatchHeader batch_header(int64_t n, int64_t tile_blocks, int64_t emit_blocks, int64_t finish_blocks,
                         int64_t render_blocks) {
  BatchHeader h{};
  h.n = n;
  h.tile_blocks = tile_blocks;
  h.emit_blocks = emit_blocks;
  h.finish_blocks = finish_blocks;
  h.render_blocks = render_blocks;
  h.layers_off = (int64_t)align256(sizeof(BatchHeader));
  h.tile_map_off = (int64_t)align256(h.layers_off + sizeof(BatchLayer) * n);
  h.emit_map_off = (int64_t)align256(h.tile_map_off + sizeof(int32_t) * tile_blocks);
  h.finish_map_off = (int64_t)align256(h.emit_map_off + sizeof(int32_t) * emit_blocks);
  h.render_map_off = (int64_t)align256(h.finish_map_off + sizeof(int32_t) * finish_blocks);
  h.grad_table_off = (int64_t)align256(h.render_map_off + sizeof(int32_t) * render_blocks);
  h.readback_off = (int64_t)align256(h.grad_table_off + sizeof(void*) * n);
  h.total = (int64_t)align256(h.readback_off + sizeof(BatchReadback) * n);
  return h;
}

// A pointer the kernel read from memory (the plan) is generic to the compiler, which then emits
// flat loads and stores; flat operations count against the LDS wait counter as well, so every
// wait for an LDS read also waits for the outstanding global ones.  A cast to the global address
// space (kept opaque, so that the compiler does not fold it with the cast back) lets the
// compiler emit global instructions.  For pointers that are uniform across the wave.
template <typename T>
__device__ inline T* glob(T* q) {
  __attribute__((address_space(1))) T* g = (__attribute__((address_space(1))) T*)q;
  asm("" : "+s"(g));
  return (T*)g;
}

// Layer l of the plan with its pointers marked global (all of them address device memory).
__device__ inline BatchLayer global_layer(const BatchLayer& src) {
  BatchLayer ly = src;
  ly.row_coords = glob(ly.row_coords);
  ly.col_coords = glob(ly.col_coords);
  ly.mu = glob(ly.mu);
  ly.chol_raw = glob(ly.chol_raw);
  ly.amp = glob(ly.amp);
  ly.delta = glob(ly.delta);
  ly.tile_ptr = glob(ly.tile_ptr);
  ly.num_pairs = glob(ly.num_pairs);
  ly.ids = glob(ly.ids);
  ly.fws = glob(ly.fws);
  ly.bws = glob(ly.bws);
  ly.d_mu = glob(ly.d_mu);
  ly.d_chol_raw = glob(ly.d_chol_raw);
  ly.d_amp = glob(ly.d_amp);
  ly.mo.base = glob(ly.mo.base);
  ly.mo.merged = glob(ly.mo.merged);
  return ly;
}

__device__ inline BatchLayer batch_layer(const uint8_t* plan, int64_t map_off, int64_t* block0_sel, int which,
                                         uint32_t blk, int32_t* index = nullptr) {
  const BatchHeader* h = reinterpret_cast<const BatchHeader*>(plan);
  const int32_t l = reinterpret_cast<const int32_t*>(plan + map_off)[blk];
  const BatchLayer& ly = reinterpret_cast<const BatchLayer*>(plan + h->layers_off)[l];
  *block0_sel = which == 0   ? ly.tile_block0
                : which == 1 ? ly.emit_block0
                : which == 2 ? ly.finish_block0
                             : ly.render_block0;
  if (index) *index = l;
  return global_layer(ly);
}

__global__ __launch_bounds__(kBinThreads) void k_bin_batch(const uint8_t* __restrict__ plan) {
  const BatchHeader* h = reinterpret_cast<const BatchHeader*>(plan);
  const BatchLayer ly = global_layer(reinterpret_cast<const BatchLayer*>(plan + h->layers_off)[blockIdx.x]);
  const Problem p = ly.p;
  const FwdLayout L = ly.fl;
  __shared__ uint32_t mlds[kMaskLdsWords];
  bin_body<true>(p, ly.mu, ly.chol_raw, ly.amp, ly.tile_ptr, ly.num_pairs, ly.fws, L, mlds);
}

__global__ __launch_bounds__(kEmitThreads) void k_emit_batch(const uint8_t* __restrict__ plan) {
  const BatchHeader* h = reinterpret_cast<const BatchHeader*>(plan);
  int64_t b0;
  const BatchLayer ly = batch_layer(plan, h->emit_map_off, &b0, 1, blockIdx.x);
  const Problem p = ly.p;
  if (p.W > 0) return;  // blocks kept for a capacity on the emission path; k is on the mask path
  const FwdLayout L = ly.fl;
  emit_body<false, kEmitLanesBatch, 2>(
      p, ly.mu, ly.amp, ly.fws, L, ly.tile_ptr, ly.ids, ly.capacity,
      (((int64_t)blockIdx.x - b0) * (kEmitThreads / 64) + wave_id()) * (64 / kEmitLanesBatch));
}

// Layers rendered tile by tile (BatchLayer::pair_render == 0: 32x32 tiles, or 16x16 tiles whose
// capacity reaches the emission path), over the tile map; the other layers' blocks return.
__global__ __launch_bounds__(kTileThreads) void k_render16_batch(const uint8_t* __restrict__ plan) {
  const BatchHeader* h = reinterpret_cast<const BatchHeader*>(plan);
  int64_t b0;
  const uint32_t blk = blockIdx.x;
  const BatchLayer ly = batch_layer(plan, h->tile_map_off, &b0, 0, blk);
  if (ly.pair_render) return;
  const Problem p = ly.p;
  render16_body(p, ly.row_coords, ly.col_coords, reinterpret_cast<const GaussEval*>(ly.fws + ly.fl.eval),
                ly.tile_ptr, ly.ids, ly.capacity, ly.delta, ly.fws,
                reinterpret_cast<const uint32_t*>(ly.fws + ly.fl.rowmask),
                reinterpret_cast<const uint32_t*>(ly.fws + ly.fl.colmask),
                sub_tile(p, (int64_t)blk - b0, wave_id()), nullptr, nullptr, 0, 1,
                reinterpret_cast<float*>(ly.fws + ly.fl.bsq), ly.mo);
}

// Layers rendered by tile pairs (16x16 tiles on the mask path at every k up to the capacity):
// a pair of horizontally adjacent tiles a wave, R x ceil(C / 2) pairs row-major, over the
// render map (which lists only these layers).
__global__ __launch_bounds__(kTileThreads) void k_render16x2_batch(const uint8_t* __restrict__ plan) {
  const BatchHeader* h = reinterpret_cast<const BatchHeader*>(plan);
  int64_t b0;
  const uint32_t blk = blockIdx.x;
  const BatchLayer ly = batch_layer(plan, h->render_map_off, &b0, 3, blk);
  const Problem p = ly.p;
  const int32_t cp = (p.C + 1) / 2;
  const int64_t pi = ((int64_t)blk - b0) * (kTileThreads / 64) + wave_id();
  if (pi >= (int64_t)p.R * cp) return;
  const int32_t tr = (int32_t)pi / cp, tc = 2 * ((int32_t)pi - tr * cp);
  render16x2_body<true>(p, ly.row_coords, ly.col_coords, reinterpret_cast<const GaussEval*>(ly.fws + ly.fl.eval),
                  ly.tile_ptr, ly.ids, ly.capacity, ly.delta, ly.fws,
                  reinterpret_cast<const uint32_t*>(ly.fws + ly.fl.rowmask),
                  reinterpret_cast<const uint32_t*>(ly.fws + ly.fl.colmask), tr, tc,
                  reinterpret_cast<float*>(ly.fws + ly.fl.bsq), ly.mo);
}

// Eight waves per SIMD: the batch's dense-tile body fits 64 VGPRs without spilling, and the
// eighth wave hides more of each tile's load chain (cfg4: 397 -> 383 us).
template <bool kMaskClamp>
__global__ __launch_bounds__(kTileThreads) __attribute__((amdgpu_waves_per_eu(8))) void k_bwd16_batch(const uint8_t* __restrict__ plan) {
  const BatchHeader* h = reinterpret_cast<const BatchHeader*>(plan);
  int64_t b0;
  int32_t l;
  const uint32_t blk = blockIdx.x;
  const BatchLayer ly = batch_layer(plan, h->tile_map_off, &b0, 0, blk, &l);
  const Problem p = ly.p;
  const BwdLayout L = ly.bl;
  const int64_t T = (int64_t)p.R * p.C;
  const int64_t P = ly.tile_ptr[T];  // pairs beyond the id capacity were never emitted
  const float* grad = glob(reinterpret_cast<const float* const*>(plan + h->grad_table_off)[l]);
  bwd16_body<int64_t, int64_t, true, kMaskClamp, true, true>(p, grad, ly.row_coords, ly.col_coords, ly.mu, ly.chol_raw,
                               reinterpret_cast<const GaussEval*>(ly.fws + ly.fl.eval),
                               ly.tile_ptr, ly.ids, P < ly.capacity ? P : ly.capacity, ly.bws, L,
                               sub_tile(p, (int64_t)blk - b0, wave_id()));
}

// dL/d(delta) pointers of layers base .. base + count - 1 (count <= kPtrChunk), passed by value.
constexpr int kPtrChunk = 256;
struct PtrChunk {
  const float* p[kPtrChunk];
};

__global__ __launch_bounds__(kPtrChunk) void k_batch_set_grads(uint8_t* plan, PtrChunk chunk, int32_t base,
                                                               int32_t count) {
  const BatchHeader* h = reinterpret_cast<const BatchHeader*>(plan);
  if ((int32_t)threadIdx.x < count)
    reinterpret_cast<const float**>(plan + h->grad_table_off)[base + threadIdx.x] = chunk.p[threadIdx.x];
}

// One workgroup per layer: forward | backward status bits, the pair count and the sum of
// delta-W^2 over the render's 16x16 blocks (in double, a fixed order: thread-strided sums, then
// a tree), into the read-back area; clear != 0 resets the status words.
__global__ __launch_bounds__(256) void k_batch_read(uint8_t* plan, int32_t clear) {
  const BatchHeader* h = reinterpret_cast<const BatchHeader*>(plan);
  const int64_t l = blockIdx.x;
  if (l >= h->n) return;
  const BatchLayer& ly = reinterpret_cast<const BatchLayer*>(plan + h->layers_off)[l];
  const Problem& p = ly.p;
  const int64_t nb = (int64_t)p.R * p.C * (p.tile_out == 32 ? 4 : 1);
  const float* bsq = reinterpret_cast<const float*>(ly.fws + ly.fl.bsq);
  double v = 0.0;
  for (int64_t i = threadIdx.x; i < nb; i += blockDim.x) v += (double)bsq[i];
  __shared__ double part[256];
  part[threadIdx.x] = v;
  __syncthreads();
  for (int o = 128; o >= 1; o >>= 1) {
    if ((int)threadIdx.x < o) part[threadIdx.x] += part[threadIdx.x + o];
    __syncthreads();
  }
  if (threadIdx.x != 0) return;
  WsHeader* fh = reinterpret_cast<WsHeader*>(ly.fws);
  WsHeader* bh = reinterpret_cast<WsHeader*>(ly.bws);
  BatchReadback r;
  r.status = fh->status | (bh ? bh->status : 0u);
  r.pad = 0u;
  r.pairs = *ly.num_pairs;
  r.delta_sumsq = part[0];
  r.pad2 = 0.0;
  reinterpret_cast<BatchReadback*>(plan + h->readback_off)[l] = r;
  if (clear) {
    fh->status = 0u;
    if (bh) bh->status = 0u;
  }
}

__global__ __launch_bounds__(kTileThreads) void k_finish_batch(const uint8_t* __restrict__ plan) {
  const BatchHeader* h = reinterpret_cast<const BatchHeader*>(plan);
  int64_t b0;
  const BatchLayer ly = batch_layer(plan, h->finish_map_off, &b0, 2, blockIdx.x);
  const Problem p = ly.p;
  const BwdLayout L = ly.bl;
  finish_body(p, ly.chol_raw, ly.amp, ly.d_mu, ly.d_chol_raw, ly.d_amp, ly.bws, L,
              ((int64_t)blockIdx.x - b0) * kTileThreads + threadIdx.x, ly.mu,
              reinterpret_cast<const float4*>(ly.fws + ly.fl.cov), reinterpret_cast<const float2*>(ly.fws + ly.fl.lfac),
              0, ly.grad_scale);
}

template <typename TP, typename GI, bool kTS, bool kMC>
void launch_bwd16(const Problem& p, int32_t xh, hipStream_t st, const float* grad, const float* rc,
                  const float* cc, const float* mu, const float* raw, const GaussEval* ev, const TP* tp,
                  const GI* gi, int64_t num_pairs, uint8_t* ws, const BwdLayout& L, const int32_t* heavy_list,
                  const uint32_t* heavy_count, const float4* dcoef = nullptr, float* dgrad = nullptr) {
  // heavy-tile kernels for the int64 saved state (FieldPlan, the autograd functions)
  constexpr bool kCanHeavy = std::is_same<TP, int64_t>::value && std::is_same<GI, int64_t>::value;
  if constexpr (kCanHeavy) {
    if (xh > 0) {
      Problem q = p;
      q.heavy = kHeavyTile;
      if constexpr (!kTS) {
        if (ev && dgrad) {  // gf_backward_direct on a field with heavy tiles
          hipLaunchKernelGGL((k_bwd16<TP, GI, false, kMC, true, true, true>), dim3((unsigned)(xh + quad_grid(p))),
                             dim3(kTileThreads), 0, st, q, grad, rc, cc, mu, raw, ev, tp, gi, num_pairs, ws, L,
                             heavy_list, heavy_count, xh, dcoef, dgrad);
          return;
        }
      }
      hipLaunchKernelGGL((k_bwd16<TP, GI, kTS, kMC, true>), dim3((unsigned)(xh + quad_grid(p))),
                         dim3(kTileThreads), 0, st, q, grad, rc, cc, mu, raw, ev, tp, gi, num_pairs, ws, L,
                         heavy_list, heavy_count, xh, nullptr, nullptr);
      return;
    }
  }
  Problem q = p;
  q.heavy = 0;
  if constexpr (kCanHeavy && !kTS) {
    if (ev && dgrad) {  // gf_backward_direct: gradients straight into dgrad
      hipLaunchKernelGGL((k_bwd16<TP, GI, false, kMC, false, true, true>), dim3((unsigned)quad_grid(p)),
                         dim3(kTileThreads), 0, st, q, grad, rc, cc, mu, raw, ev, tp, gi, num_pairs, ws, L,
                         heavy_list, heavy_count, 0, dcoef, dgrad);
      return;
    }
  }
  if constexpr (kCanHeavy) {
    if (ev) {  // the forward's constants (FieldPlan, the autograd functions)
      hipLaunchKernelGGL((k_bwd16<TP, GI, kTS, kMC, false, true>), dim3((unsigned)quad_grid(p)), dim3(kTileThreads),
                         0, st, q, grad, rc, cc, mu, raw, ev, tp, gi, num_pairs, ws, L, heavy_list, heavy_count, 0,
                         nullptr, nullptr);
      return;
    }
  }
  hipLaunchKernelGGL((k_bwd16<TP, GI, kTS, kMC, false>), dim3((unsigned)quad_grid(p)), dim3(kTileThreads), 0, st,
                     q, grad, rc, cc, mu, raw, ev, tp, gi, num_pairs, ws, L, heavy_list, heavy_count, 0, nullptr,
                     nullptr);
}

// Tiles of several Gaussians (P >= 8 T: a wave makes two or more rounds on average) take the
// transposing moment reduction (fewer instructions); sparse ones the row sums (shorter chain).
// cfg5 (11.6 pairs a tile) 34.6 -> 29.8 us with the transposing form; at 4.5 pairs a tile
// (cfg2) it would cost the one-launch form below.
bool bwd_dense(const Problem& p, int64_t num_pairs) { return num_pairs >= 8 * (int64_t)p.R * p.C; }
// The one-launch backward's limit: fewer than 16 pairs a tile.
bool direct_pairs_fit(const Problem& p, int64_t num_pairs) { return num_pairs < 16 * (int64_t)p.R * p.C; }

template <typename TP, typename GI>
void launch_bwd(const Problem& p, dim3 grid, hipStream_t st, const float* grad, const float* rc,
                const float* cc, const float* mu, const float* raw, const GaussEval* ev,
                const void* tile_ptr, const void* gids, int64_t num_pairs, uint8_t* ws,
                const BwdLayout& L, const int32_t* heavy_list, const uint32_t* heavy_count,
                const float4* dcoef = nullptr, float* dgrad = nullptr) {
  // (the one-launch gradients, dgrad, take the row sums: up to 16 pairs a tile)
  const bool dense = !dgrad && bwd_dense(p, num_pairs);
  // heavy-tile workgroups only with the forward's tile list (the forward workspace)
  const int32_t xh = heavy_list ? heavy_grid(p, num_pairs) : 0;
  const TP* tp = reinterpret_cast<const TP*>(tile_ptr);
  const GI* gi = reinterpret_cast<const GI*>(gids);
  if (quad_tiles(p)) {
    if (p.mask_clamp && dense)
      launch_bwd16<TP, GI, true, true>(p, xh, st, grad, rc, cc, mu, raw, ev, tp, gi, num_pairs, ws, L, heavy_list,
                                       heavy_count);
    else if (p.mask_clamp)
      launch_bwd16<TP, GI, false, true>(p, xh, st, grad, rc, cc, mu, raw, ev, tp, gi, num_pairs, ws, L, heavy_list,
                                        heavy_count, dcoef, dgrad);
    else if (dense)
      launch_bwd16<TP, GI, true, false>(p, xh, st, grad, rc, cc, mu, raw, ev, tp, gi, num_pairs, ws, L, heavy_list,
                                        heavy_count);
    else
      launch_bwd16<TP, GI, false, false>(p, xh, st, grad, rc, cc, mu, raw, ev, tp, gi, num_pairs, ws, L,
                                         heavy_list, heavy_count, dcoef, dgrad);
  } else
    hipLaunchKernelGGL((k_bwd_any<TP, GI>), grid, dim3(kTileThreads), 0, st, p, grad, rc, cc, mu, raw, ev,
                       reinterpret_cast<const TP*>(tile_ptr), reinterpret_cast<const GI*>(gids),
                       num_pairs, ws, L);
}

// ------------------------------------------------------------------------------------------
// Allocation-free backward (gf_backward_noalloc).  Its workspace -- the header with the status
// word and the S x K accumulator slots -- lives in this static device array, one copy per GPU,
// held until the process ends.  4 MiB: K up to 131,064 Gaussians for S = 1 (fewer than 2048 tiles),
// 32,766 for S = 4, 16,383 for S = 8 and 4,095 for S = 32.
constexpr size_t kNoAllocScratchBytes = size_t(4) << 20;

// Clears n 16-byte words (a fill kernel rather than hipMemsetAsync, which must not be recorded
// into the HIP graphs a caller of the allocation-free entry may capture).
__global__ __launch_bounds__(256) void k_fill_zero(uint4* __restrict__ p, int64_t n) {
  for (int64_t i = (int64_t)blockIdx.x * blockDim.x + threadIdx.x; i < n; i += (int64_t)gridDim.x * blockDim.x)
    p[i] = make_uint4(0u, 0u, 0u, 0u);
}

// Clears a workspace's status word (a kernel, ordered after a read-back copy on the stream).
// The one-launch backward's gradients out of their slots (dgrad[K][8]: d_amp, d_mu x2,
// d_chol_raw x3) into the caller's arrays, clearing each slot for the next backward on the same
// forward (gf_backward_train).
__global__ __launch_bounds__(256) void k_slots_out(float4* __restrict__ slots, int64_t K, float* __restrict__ d_mu,
                                                   float* __restrict__ d_chol_raw, float* __restrict__ d_amp) {
  const int64_t g = (int64_t)blockIdx.x * 256 + threadIdx.x;
  if (g >= K) return;
  const float4 a = slots[2 * g], b = slots[2 * g + 1];
  d_amp[g] = a.x;
  d_mu[2 * g + 0] = a.y;
  d_mu[2 * g + 1] = a.z;
  d_chol_raw[3 * g + 0] = a.w;
  d_chol_raw[3 * g + 1] = b.x;
  d_chol_raw[3 * g + 2] = b.y;
  slots[2 * g] = make_float4(0.0f, 0.0f, 0.0f, 0.0f);
  slots[2 * g + 1] = make_float4(0.0f, 0.0f, 0.0f, 0.0f);
}

__global__ __launch_bounds__(64) void k_clear_status(uint32_t* __restrict__ status) {
  if (threadIdx.x == 0) *status = 0u;
}

// Copies a workspace's status word to the caller's device word.
__global__ __launch_bounds__(64) void k_copy_status(const uint32_t* __restrict__ status, uint32_t* __restrict__ out) {
  if (threadIdx.x == 0) *out = *status;
}

// Page-locked host memory for the small host read-backs (gf_forward_bin's pair count, gf_read_status):
// a device-to-host copy into pageable memory is staged and measured about 11 us slower than one into
// page-locked memory.  One 256-byte buffer per host thread (the read-backs synchronise their stream,
// so a thread has at most one in flight), allocated at the thread's first read-back and held until
// the process ends.
thread_local void* g_pinned = nullptr;

int pinned_readback(void** out) {
  if (!g_pinned) {
    void* ptr = nullptr;
    const hipError_t e = hipHostMalloc(&ptr, 256, hipHostMallocDefault);
    if (e != hipSuccess || !ptr) return set_err(GF_E_HIP, "hipHostMalloc(256) failed: %s", hipGetErrorString(e));
    g_pinned = ptr;
  }
  *out = g_pinned;
  return GF_OK;
}

}  // namespace

static __device__ __align__(256) uint8_t scratch[kNoAllocScratchBytes];

namespace {

// The device address of `scratch` on the current device, looked up once per device with that
// device current (each GPU holds its own copy of the array at its own address).  In host code
// the name `scratch` is only a host-side stand-in: kernels get this address instead.
constexpr int kMaxDevices = 64;
std::mutex g_scratch_mutex;
void* g_scratch_ptr[kMaxDevices];

int scratch_for_current_device(void** out) {
  int dev = -1;
  GF_HIP_CHECK(hipGetDevice(&dev));
  if (dev < 0 || dev >= kMaxDevices) return set_err(GF_E_HIP, "device ordinal %d out of range", dev);
  std::lock_guard<std::mutex> lock(g_scratch_mutex);
  if (!g_scratch_ptr[dev]) {
    void* ptr = nullptr;
    const hipError_t e = hipGetSymbolAddress(&ptr, HIP_SYMBOL(scratch));
    if (e != hipSuccess || !ptr)
      return set_err(GF_E_HIP, "hipGetSymbolAddress(scratch) on device %d failed: %s", dev, hipGetErrorString(e));
    g_scratch_ptr[dev] = ptr;
  }
  *out = g_scratch_ptr[dev];
  return GF_OK;
}

}  // namespace

// ------------------------------------------------------------------------------------------
// C ABI.

extern "C" {

const char* gf_version(void) { return GF_VERSION; }
const char* gf_last_error(void) { return g_err; }

int gf_tile_grid(int64_t out_features, int64_t in_features, const gf_field_config* cfg,
                 int64_t* num_tile_rows_host, int64_t* num_tile_cols_host) {
  Problem p;
  int rc = make_problem(cfg, out_features, in_features, 0, &p);
  if (rc) return rc;
  if (num_tile_rows_host) *num_tile_rows_host = p.R;
  if (num_tile_cols_host) *num_tile_cols_host = p.C;
  return GF_OK;
}

size_t gf_forward_workspace_bytes(int64_t out_features, int64_t in_features, int64_t k,
                                  const gf_field_config* cfg) {
  Problem p;
  if (make_problem(cfg, out_features, in_features, k, &p)) return 0;
  return fwd_layout(p).total;
}

size_t gf_forward_workspace_bytes_max(int64_t out_features, int64_t in_features, int64_t k_capacity,
                                      const gf_field_config* cfg) {
  // Every condition of the mask path is an upper bound on K, so the mask path holds exactly for
  // 1 <= K <= K*; the bytes grow with K on either side of K*, and the largest need over
  // [0, k_capacity] is that of k_capacity or of min(k_capacity, K*).
  Problem p;
  if (k_capacity < 0 || make_problem(cfg, out_features, in_features, k_capacity, &p)) return 0;
  size_t most = fwd_layout(p).total;
  int64_t lo = 0, hi = std::min<int64_t>(k_capacity, kMaskMaxK);  // largest K on the mask path
  while (lo < hi) {
    const int64_t mid = lo + (hi - lo + 1) / 2;
    Problem q;
    if (make_problem(cfg, out_features, in_features, mid, &q) == GF_OK && q.W > 0)
      lo = mid;
    else
      hi = mid - 1;
  }
  if (lo > 0) {
    Problem q;
    if (make_problem(cfg, out_features, in_features, lo, &q) == GF_OK) most = std::max(most, fwd_layout(q).total);
  }
  return most;
}

size_t gf_backward_workspace_bytes(int64_t out_features, int64_t in_features, int64_t k,
                                   const gf_field_config* cfg) {
  Problem p;
  if (make_problem(cfg, out_features, in_features, k, &p)) return 0;
  return bwd_layout(p).total;
}

static int forward_bin(const gf_field_config* cfg, int64_t out_features, int64_t in_features, int64_t k,
                       const float* mu, const float* chol_raw, const float* amp, int64_t* tile_ptr,
                       int64_t* num_pairs_dev, gf_bin_info* info, void* workspace, size_t workspace_bytes,
                       void* stream, bool force_tiles, const int64_t* kdev = nullptr);

int gf_forward_bin(const gf_field_config* cfg, int64_t out_features, int64_t in_features, int64_t k,
                   const float* mu, const float* chol_raw, const float* amp, int64_t* tile_ptr,
                   int64_t* num_pairs_dev, int64_t* num_pairs_host, void* workspace,
                   size_t workspace_bytes, void* stream) {
  gf_bin_info info;
  const int rc = forward_bin(cfg, out_features, in_features, k, mu, chol_raw, amp, tile_ptr, num_pairs_dev,
                             num_pairs_host ? &info : nullptr, workspace, workspace_bytes, stream, false);
  if (rc == GF_OK && num_pairs_host) *num_pairs_host = info.num_pairs;
  return rc;
}

int gf_forward_bin_info(const gf_field_config* cfg, int64_t out_features, int64_t in_features, int64_t k,
                        const float* mu, const float* chol_raw, const float* amp, int64_t* tile_ptr,
                        int64_t* num_pairs_dev, gf_bin_info* info, void* workspace, size_t workspace_bytes,
                        void* stream) {
  if (!info) return set_err(GF_E_INVALID_ARGUMENT, "info must not be NULL");
  return forward_bin(cfg, out_features, in_features, k, mu, chol_raw, amp, tile_ptr, num_pairs_dev, info,
                     workspace, workspace_bytes, stream, false);
}

// force_tiles: bin the tiles with k_bin_tiles (tile_ptr and the chain-rule maps stored here) also
// where the render would bin them itself (tiles_in_render).  kdev: capacity mode (k is the capacity,
// the live K is *kdev; see Problem::kdev).
static int forward_bin(const gf_field_config* cfg, int64_t out_features, int64_t in_features, int64_t k,
                       const float* mu, const float* chol_raw, const float* amp, int64_t* tile_ptr,
                       int64_t* num_pairs_dev, gf_bin_info* info, void* workspace, size_t workspace_bytes,
                       void* stream, bool force_tiles, const int64_t* kdev) {
  Problem p;
  int rc = make_problem(cfg, out_features, in_features, k, &p);
  if (rc) return rc;
  p.kdev = kdev;
  const FwdLayout L = fwd_layout(p);
  if (!workspace || workspace_bytes < L.total)
    return set_err(GF_E_WORKSPACE, "forward workspace needs %zu bytes, got %zu", L.total, workspace_bytes);
  if (!tile_ptr || !num_pairs_dev) return set_err(GF_E_INVALID_ARGUMENT, "tile_ptr / num_pairs_dev must not be NULL");
  if (k > 0 && (!mu || !chol_raw)) return set_err(GF_E_INVALID_ARGUMENT, "mu / chol_raw must not be NULL");
  hipStream_t st = reinterpret_cast<hipStream_t>(stream);
  unsigned parts = 0;  // WsHeader::part entries that hold P (tiles binned in the render)
  if (p.W > 0) {
    if (!amp) return set_err(GF_E_INVALID_ARGUMENT, "amp must not be NULL");
    uint8_t* ws = reinterpret_cast<uint8_t*>(workspace);
    const unsigned lines = (unsigned)(p.R + p.C);
    const bool in_render = !force_tiles && binned_in_render(p);
    const bool split = in_render || prep_split(p);  // in_render: K <= kRowsMaxK
    const int64_t per = split ? kTilesThreads / 4 : kTilesThreads;
    const unsigned nbp = (unsigned)((k + per - 1) / per);
    const unsigned nbc = in_render ? (unsigned)((k + kCoefPerBlock - 1) / kCoefPerBlock) : 0u;
    auto prep = in_render ? k_prep<true, true> : split ? k_prep<false, true> : k_prep<false, false>;
    hipLaunchKernelGGL(prep, dim3(nbp + nbc), dim3(kTilesThreads), 0, st, p, mu, chol_raw, amp, ws, L, num_pairs_dev);
    GF_LAUNCH_CHECK("k_prep");
    if (in_render) parts = nbp;
    p.heavy = heavy_threshold(p);
    if (!in_render)
      hipLaunchKernelGGL(k_bin_tiles, dim3(lines), dim3(kTilesThreads), 0, st, p, tile_ptr, num_pairs_dev, ws, L,
                         chol_raw, amp);
  } else {
    hipLaunchKernelGGL(k_bin, dim3(1), dim3(kBinThreads), 0, st, p, mu, chol_raw, tile_ptr,
                       num_pairs_dev, reinterpret_cast<uint8_t*>(workspace), L);
  }
  GF_LAUNCH_CHECK("k_bin");
  if (info) {
    // the status word, P and the widest rectangle sit in the first 32 bytes of the header (or
    // P in the preparation workgroups' part entries after them, where the render bins the
    // tiles): one copy into page-locked memory
    void* pinned = nullptr;
    rc = pinned_readback(&pinned);
    if (rc) return rc;
    const size_t bytes = parts ? offsetof(WsHeader, pad) : offsetof(WsHeader, max_span) + sizeof(int64_t);
    GF_HIP_CHECK(hipMemcpyAsync(pinned, workspace, bytes, hipMemcpyDeviceToHost, st));
    GF_HIP_CHECK(hipStreamSynchronize(st));
    const WsHeader* h = reinterpret_cast<const WsHeader*>(pinned);
    if (parts) {
      int64_t P = 0, span = 0;
      for (unsigned b = 0; b < parts; ++b) {
        P += h->part[b][0];
        span = std::max<int64_t>(span, h->part[b][1]);
      }
      info->num_pairs = P;
      info->max_span = span;
    } else {
      info->num_pairs = h->pairs;
      info->max_span = h->max_span;
    }
    if (h->status & GF_STATUS_COUNT_MISMATCH)
      return set_err(GF_E_INTERNAL, "binning: per-tile counts disagree with per-Gaussian tile totals");
  }
  return GF_OK;
}

int gf_forward_emit(const gf_field_config* cfg, int64_t out_features, int64_t in_features, int64_t k,
                    const float* mu, const float* amp, const int64_t* tile_ptr,
                    int64_t* gaussian_ids_sorted, int64_t ids_capacity,
                    void* workspace, size_t workspace_bytes, void* stream) {
  Problem p;
  int rc = make_problem(cfg, out_features, in_features, k, &p);
  if (rc) return rc;
  const FwdLayout L = fwd_layout(p);
  if (!workspace || workspace_bytes < L.total)
    return set_err(GF_E_WORKSPACE, "forward workspace needs %zu bytes, got %zu", L.total, workspace_bytes);
  if (ids_capacity < 0 || (ids_capacity > 0 && !gaussian_ids_sorted))
    return set_err(GF_E_INVALID_ARGUMENT, "gaussian_ids_sorted / ids_capacity invalid");
  if (!tile_ptr) return set_err(GF_E_INVALID_ARGUMENT, "tile_ptr must not be NULL");
  if (k > 0 && (!mu || !amp)) return set_err(GF_E_INVALID_ARGUMENT, "mu / amp must not be NULL");
  if (k == 0 || p.W > 0) return GF_OK;  // mask path: the render reads the ids from the masks
  hipStream_t st = reinterpret_cast<hipStream_t>(stream);
  const int64_t blocks = (k + kEmitThreads / 64 - 1) / (kEmitThreads / 64);
  hipLaunchKernelGGL(k_emit, dim3((unsigned)blocks), dim3(kEmitThreads), 0, st, p, mu, amp,
                     reinterpret_cast<uint8_t*>(workspace), L, tile_ptr, gaussian_ids_sorted,
                     ids_capacity);
  GF_LAUNCH_CHECK("k_emit");
  return GF_OK;
}

static int forward_render(const gf_field_config* cfg, int64_t out_features, int64_t in_features, int64_t k,
                          const float* row_coords, const float* col_coords, int64_t* tile_ptr,
                          int64_t* gaussian_ids_sorted, int64_t ids_capacity, float* delta, void* workspace,
                          size_t workspace_bytes, void* stream, const int64_t* kdev);

int gf_forward_render(const gf_field_config* cfg, int64_t out_features, int64_t in_features, int64_t k,
                      const float* row_coords, const float* col_coords, int64_t* tile_ptr,
                      int64_t* gaussian_ids_sorted, int64_t ids_capacity,
                      float* delta, void* workspace, size_t workspace_bytes, void* stream) {
  return forward_render(cfg, out_features, in_features, k, row_coords, col_coords, tile_ptr, gaussian_ids_sorted,
                        ids_capacity, delta, workspace, workspace_bytes, stream, nullptr);
}

static int forward_render(const gf_field_config* cfg, int64_t out_features, int64_t in_features, int64_t k,
                          const float* row_coords, const float* col_coords, int64_t* tile_ptr,
                          int64_t* gaussian_ids_sorted, int64_t ids_capacity, float* delta, void* workspace,
                          size_t workspace_bytes, void* stream, const int64_t* kdev) {
  Problem p;
  int rc = make_problem(cfg, out_features, in_features, k, &p);
  if (rc) return rc;
  p.kdev = kdev;
  const int64_t T = (int64_t)p.R * p.C;
  const FwdLayout L = fwd_layout(p);
  if (!workspace || workspace_bytes < L.total)
    return set_err(GF_E_WORKSPACE, "forward workspace needs %zu bytes, got %zu", L.total, workspace_bytes);
  if (!row_coords || !col_coords || !tile_ptr || !delta)
    return set_err(GF_E_INVALID_ARGUMENT, "coords / tile_ptr / delta must not be NULL");
  if (ids_capacity < 0 || (ids_capacity > 0 && !gaussian_ids_sorted))
    return set_err(GF_E_INVALID_ARGUMENT, "gaussian_ids_sorted / ids_capacity invalid");
  hipStream_t st = reinterpret_cast<hipStream_t>(stream);
  uint8_t* ws = reinterpret_cast<uint8_t*>(workspace);
  const GaussEval* ev = reinterpret_cast<const GaussEval*>(ws + L.eval);
  if (quad_render(p)) {
    if (rows_in_render(p)) {
      const int32_t cp = (p.C + 1) / 2, G = (cp + kRowsThreads / 64 - 1) / (kRowsThreads / 64);
      hipLaunchKernelGGL(k_render16x2_rows, dim3((unsigned)((int64_t)p.R * G)), dim3(kRowsThreads), 0, st, p,
                         row_coords, col_coords, ev, tile_ptr, gaussian_ids_sorted, ids_capacity, delta, ws,
                         reinterpret_cast<const int4*>(ws + L.rect));
      GF_LAUNCH_CHECK("k_render16x2_rows");
      return GF_OK;
    }
    const bool binned_here = tiles_in_render(p);
    const int32_t xh = heavy_grid(p, ids_capacity);
    p.heavy = xh > 0 ? kHeavyTile : 0;
    if (p.tile_out == 16 && p.tile_in == 16 && p.W > 0 && !binned_here) {
      const int64_t pairs = (int64_t)p.R * ((p.C + 1) / 2);
      const unsigned pair_blocks = (unsigned)((pairs + kTileThreads / 64 - 1) / (kTileThreads / 64));
      if (xh == 0) {
        hipLaunchKernelGGL(k_render16x2, dim3(pair_blocks), dim3(kTileThreads), 0, st, p, row_coords, col_coords, ev,
                           tile_ptr, gaussian_ids_sorted, ids_capacity, delta, ws,
                           reinterpret_cast<const uint32_t*>(ws + L.rowmask),
                           reinterpret_cast<const uint32_t*>(ws + L.colmask));
        GF_LAUNCH_CHECK("k_render16x2");
      } else {
        hipLaunchKernelGGL(k_render16x2_heavy, dim3((unsigned)xh + pair_blocks), dim3(kTileThreads), 0, st, p,
                           row_coords, col_coords, ev, tile_ptr, gaussian_ids_sorted, ids_capacity, delta, ws,
                           reinterpret_cast<const uint32_t*>(ws + L.rowmask),
                           reinterpret_cast<const uint32_t*>(ws + L.colmask),
                           reinterpret_cast<const int32_t*>(ws + L.fill), xh);
        GF_LAUNCH_CHECK("k_render16x2_heavy");
      }
      return GF_OK;
    }
    hipLaunchKernelGGL(xh > 0 ? k_render16<true> : k_render16<false>, dim3((unsigned)(xh + quad_grid(p))),
                       dim3(kTileThreads), 0, st, p, row_coords, col_coords, ev, tile_ptr, gaussian_ids_sorted,
                       ids_capacity, delta, ws, reinterpret_cast<const uint32_t*>(ws + L.rowmask),
                       reinterpret_cast<const uint32_t*>(ws + L.colmask),
                       binned_here ? reinterpret_cast<const int4*>(ws + L.rect) : nullptr,
                       binned_here ? tile_ptr : nullptr, reinterpret_cast<const int32_t*>(ws + L.fill), xh);
  }
  else
    hipLaunchKernelGGL(k_render_any, dim3((unsigned)T), dim3(kTileThreads), 0, st, p, row_coords,
                       col_coords, ev, tile_ptr, gaussian_ids_sorted, ids_capacity, delta, ws);
  GF_LAUNCH_CHECK("k_render");
  return GF_OK;
}

int gf_forward(const gf_field_config* cfg, int64_t out_features, int64_t in_features, int64_t k,
               const float* row_coords, const float* col_coords, const float* mu, const float* chol_raw,
               const float* amp, int64_t* tile_ptr, int64_t* num_pairs_dev, int64_t* gaussian_ids_sorted,
               int64_t ids_capacity, float* delta, void* workspace, size_t workspace_bytes, void* stream) {
  int rc = gf_forward_bin(cfg, out_features, in_features, k, mu, chol_raw, amp, tile_ptr, num_pairs_dev, nullptr,
                          workspace, workspace_bytes, stream);
  if (rc) return rc;
  rc = gf_forward_emit(cfg, out_features, in_features, k, mu, amp, tile_ptr, gaussian_ids_sorted, ids_capacity,
                       workspace, workspace_bytes, stream);
  if (rc) return rc;
  return gf_forward_render(cfg, out_features, in_features, k, row_coords, col_coords, tile_ptr,
                           gaussian_ids_sorted, ids_capacity, delta, workspace, workspace_bytes, stream);
}

static int backward_reduce(const gf_field_config* cfg, int64_t out_features, int64_t in_features, int64_t k,
                           const float* grad_delta, const float* row_coords, const float* col_coords,
                           const float* mu, const float* chol_raw, const void* tile_ptr, int32_t tile_ptr_is_int64,
                           const void* gaussian_ids, int32_t ids_is_int64, int64_t num_pairs,
                           const void* forward_workspace, void* workspace, size_t workspace_bytes, void* stream,
                           const int64_t* kdev, const int64_t* pdev);

int gf_backward_reduce(const gf_field_config* cfg, int64_t out_features, int64_t in_features, int64_t k,
                       const float* grad_delta, const float* row_coords, const float* col_coords,
                       const float* mu, const float* chol_raw, const void* tile_ptr,
                       int32_t tile_ptr_is_int64, const void* gaussian_ids, int32_t ids_is_int64,
                       int64_t num_pairs, const void* forward_workspace, void* workspace,
                       size_t workspace_bytes, void* stream) {
  return backward_reduce(cfg, out_features, in_features, k, grad_delta, row_coords, col_coords, mu, chol_raw,
                         tile_ptr, tile_ptr_is_int64, gaussian_ids, ids_is_int64, num_pairs, forward_workspace,
                         workspace, workspace_bytes, stream, nullptr, nullptr);
}

// kdev / pdev: capacity mode (k is the capacity; see Problem::kdev); num_pairs then only bounds
// the launch (its heavy-tile and dense-tile choices).
static int backward_reduce(const gf_field_config* cfg, int64_t out_features, int64_t in_features, int64_t k,
                           const float* grad_delta, const float* row_coords, const float* col_coords,
                           const float* mu, const float* chol_raw, const void* tile_ptr, int32_t tile_ptr_is_int64,
                           const void* gaussian_ids, int32_t ids_is_int64, int64_t num_pairs,
                           const void* forward_workspace, void* workspace, size_t workspace_bytes, void* stream,
                           const int64_t* kdev, const int64_t* pdev) {
  Problem p;
  int rc = make_problem(cfg, out_features, in_features, k, &p);
  if (rc) return rc;
  p.kdev = kdev;
  p.pdev = pdev;
  const int64_t T = (int64_t)p.R * p.C;
  const BwdLayout L = bwd_layout(p);
  if (!workspace || workspace_bytes < L.total)
    return set_err(GF_E_WORKSPACE, "backward workspace needs %zu bytes, got %zu", L.total, workspace_bytes);
  if (num_pairs < 0) return set_err(GF_E_INVALID_ARGUMENT, "num_pairs must be non-negative");
  if (!grad_delta || !row_coords || !col_coords || !tile_ptr)
    return set_err(GF_E_INVALID_ARGUMENT, "grad_delta / coords / tile_ptr must not be NULL");
  if (num_pairs > 0 && !gaussian_ids) return set_err(GF_E_INVALID_ARGUMENT, "gaussian_ids must not be NULL");
  if (k > 0 && (!mu || !chol_raw)) return set_err(GF_E_INVALID_ARGUMENT, "mu / chol_raw must not be NULL");
  hipStream_t st = reinterpret_cast<hipStream_t>(stream);
  uint8_t* ws = reinterpret_cast<uint8_t*>(workspace);
  const uint8_t* fws = reinterpret_cast<const uint8_t*>(forward_workspace);
  const GaussEval* ev = fws ? reinterpret_cast<const GaussEval*>(fws + fwd_layout(p).eval) : nullptr;
  // The heavy-tile list comes with the forward workspace of the forward that binned these tiles.
  const int32_t* heavy_list = fws ? reinterpret_cast<const int32_t*>(fws + fwd_layout(p).fill) : nullptr;
  const uint32_t* heavy_count = fws ? &reinterpret_cast<const WsHeader*>(fws)->heavy : nullptr;
  const dim3 grid((unsigned)T);
  if (tile_ptr_is_int64 && ids_is_int64)
    launch_bwd<int64_t, int64_t>(p, grid, st, grad_delta, row_coords, col_coords, mu, chol_raw, ev, tile_ptr, gaussian_ids, num_pairs, ws, L, heavy_list, heavy_count);
  else if (tile_ptr_is_int64)
    launch_bwd<int64_t, int32_t>(p, grid, st, grad_delta, row_coords, col_coords, mu, chol_raw, ev, tile_ptr, gaussian_ids, num_pairs, ws, L, heavy_list, heavy_count);
  else if (ids_is_int64)
    launch_bwd<int32_t, int64_t>(p, grid, st, grad_delta, row_coords, col_coords, mu, chol_raw, ev, tile_ptr, gaussian_ids, num_pairs, ws, L, heavy_list, heavy_count);
  else
    launch_bwd<int32_t, int32_t>(p, grid, st, grad_delta, row_coords, col_coords, mu, chol_raw, ev, tile_ptr, gaussian_ids, num_pairs, ws, L, heavy_list, heavy_count);
  GF_LAUNCH_CHECK("k_bwd");
  return GF_OK;
}

static int backward_finish(const gf_field_config* cfg, int64_t out_features, int64_t in_features, int64_t k,
                           const float* chol_raw, const float* amp, float* d_mu, float* d_chol_raw, float* d_amp,
                           const void* forward_workspace, void* workspace, size_t workspace_bytes, void* stream,
                           int32_t ostride, const int64_t* kdev = nullptr);

int gf_backward_finish(const gf_field_config* cfg, int64_t out_features, int64_t in_features, int64_t k,
                       const float* chol_raw, const float* amp, float* d_mu, float* d_chol_raw,
                       float* d_amp, const void* forward_workspace, void* workspace, size_t workspace_bytes,
                       void* stream) {
  return backward_finish(cfg, out_features, in_features, k, chol_raw, amp, d_mu, d_chol_raw, d_amp,
                         forward_workspace, workspace, workspace_bytes, stream, 0);
}

// gf_backward_finish with the outputs' per-Gaussian stride (finish_body's ostride); kdev: capacity mode.
static int backward_finish(const gf_field_config* cfg, int64_t out_features, int64_t in_features, int64_t k,
                           const float* chol_raw, const float* amp, float* d_mu, float* d_chol_raw, float* d_amp,
                           const void* forward_workspace, void* workspace, size_t workspace_bytes, void* stream,
                           int32_t ostride, const int64_t* kdev) {
  Problem p;
  int rc = make_problem(cfg, out_features, in_features, k, &p);
  if (rc) return rc;
  p.kdev = kdev;
  const BwdLayout L = bwd_layout(p);
  if (!workspace || workspace_bytes < L.total)
    return set_err(GF_E_WORKSPACE, "backward workspace needs %zu bytes, got %zu", L.total, workspace_bytes);
  if (k == 0) return GF_OK;
  if (!chol_raw || !amp || !d_mu || !d_chol_raw || !d_amp)
    return set_err(GF_E_INVALID_ARGUMENT, "parameter / gradient pointers must not be NULL");
  hipStream_t st = reinterpret_cast<hipStream_t>(stream);
  const unsigned blocks = (unsigned)((k * p.S + kTileThreads - 1) / kTileThreads);
  const uint8_t* fws = reinterpret_cast<const uint8_t*>(forward_workspace);
  const FwdLayout FL = fwd_layout(p);
  hipLaunchKernelGGL(k_bwd_finish, dim3(blocks), dim3(kTileThreads), 0, st, p, chol_raw, amp, d_mu,
                     d_chol_raw, d_amp, reinterpret_cast<uint8_t*>(workspace), L,
                     fws ? reinterpret_cast<const float4*>(fws + FL.cov) : nullptr,
                     fws ? reinterpret_cast<const float2*>(fws + FL.lfac) : nullptr, ostride);
  GF_LAUNCH_CHECK("k_bwd_finish");
  return GF_OK;
}

int gf_backward(const gf_field_config* cfg, int64_t out_features, int64_t in_features, int64_t k,
                const float* grad_delta, const float* row_coords, const float* col_coords,
                const float* mu, const float* chol_raw, const float* amp, const void* tile_ptr,
                int32_t tile_ptr_is_int64, const void* gaussian_ids, int32_t ids_is_int64,
                int64_t num_pairs, float* d_mu, float* d_chol_raw, float* d_amp,
                const void* forward_workspace, void* workspace, size_t workspace_bytes, void* stream) {
  if (k > 0 && !amp) return set_err(GF_E_INVALID_ARGUMENT, "amp must not be NULL");
  int rc = gf_backward_reduce(cfg, out_features, in_features, k, grad_delta, row_coords, col_coords,
                              mu, chol_raw, tile_ptr, tile_ptr_is_int64, gaussian_ids, ids_is_int64,
                              num_pairs, forward_workspace, workspace, workspace_bytes, stream);
  if (rc) return rc;
  return gf_backward_finish(cfg, out_features, in_features, k, chol_raw, amp, d_mu, d_chol_raw, d_amp,
                            forward_workspace, workspace, workspace_bytes, stream);
}

// gf_backward_direct runs one launch where the binning stored the chain-rule maps (the mask
// path) and the tiles take the row-sum kernels: 16x16 or 32x32 tiles, sparse (heavy tiles
// included: their four-wave workgroups add into the slots too).  The direct gradients have one
// slot per Gaussian, so a Gaussian's atomics cannot be spread over stripes: on grids of 8192
// tiles or more, whose Gaussians can touch thousands of tiles, it runs the reduction and the
// finish, which writes the same gradients, unless the binning's widest rectangle is known to be
// under kDirectMaxSpan tiles.  One wide Gaussian serialises the direct kernel's atomics on its
// slot, about 10 ns a tile.  Measured at cfg3's grid with one centred Gaussian of growing rectangle:
//   tiles of the rectangle    15    256    625    1369   2401   6400
//   one launch, us            9.3   10.8   15.3   23.7   36.6   85.1
//   reduction + finish, us    11.7  11.6   11.7   13.8   17.0   27.3
// so where the binning's widest rectangle is known (gf_bin_info.max_span; negative: not known)
// one of kDirectMaxSpan tiles or more sends the call to the reduction + finish.
constexpr int64_t kDirectMaxSpan = 320;
bool direct_one_launch(const Problem& p, int64_t num_pairs, int64_t max_span) {
  const bool small_grid = (int64_t)p.R * p.C < 8192;
  return p.W > 0 && quad_tiles(p) && (small_grid || max_span >= 0) && direct_pairs_fit(p, num_pairs) &&
         max_span < kDirectMaxSpan;
}

int gf_backward_direct_launches(const gf_field_config* cfg, int64_t out_features, int64_t in_features, int64_t k,
                                int64_t num_pairs, int64_t max_span) {
  Problem p;
  int rc = make_problem(cfg, out_features, in_features, k, &p);
  if (rc) return -rc;
  return direct_one_launch(p, num_pairs, max_span) && k > 0 ? 1 : 2;
}

size_t gf_forward_grads_offset(int64_t out_features, int64_t in_features, int64_t k,
                               const gf_field_config* cfg) {
  Problem p;
  if (make_problem(cfg, out_features, in_features, k, &p)) return 0;
  return fwd_layout(p).dgrad;
}

static int backward_direct(const gf_field_config* cfg, int64_t out_features, int64_t in_features, int64_t k,
                           const float* grad_delta, const float* row_coords, const float* col_coords,
                           const float* mu, const float* chol_raw, const float* amp, const int64_t* tile_ptr,
                           const int64_t* gaussian_ids, int64_t num_pairs, int64_t max_span, void* forward_workspace,
                           size_t forward_workspace_bytes, void* workspace, size_t workspace_bytes, void* stream,
                           const int64_t* kdev, const int64_t* pdev, bool* one_launch = nullptr);

int gf_backward_direct(const gf_field_config* cfg, int64_t out_features, int64_t in_features, int64_t k,
                       const float* grad_delta, const float* row_coords, const float* col_coords,
                       const float* mu, const float* chol_raw, const float* amp, const int64_t* tile_ptr,
                       const int64_t* gaussian_ids, int64_t num_pairs, int64_t max_span, void* forward_workspace,
                       size_t forward_workspace_bytes, void* workspace, size_t workspace_bytes, void* stream) {
  return backward_direct(cfg, out_features, in_features, k, grad_delta, row_coords, col_coords, mu, chol_raw, amp,
                         tile_ptr, gaussian_ids, num_pairs, max_span, forward_workspace, forward_workspace_bytes,
                         workspace, workspace_bytes, stream, nullptr, nullptr);
}

// one_launch (optional): set to whether the one-launch kernel ran.
static int backward_direct(const gf_field_config* cfg, int64_t out_features, int64_t in_features, int64_t k,
                           const float* grad_delta, const float* row_coords, const float* col_coords,
                           const float* mu, const float* chol_raw, const float* amp, const int64_t* tile_ptr,
                           const int64_t* gaussian_ids, int64_t num_pairs, int64_t max_span, void* forward_workspace,
                           size_t forward_workspace_bytes, void* workspace, size_t workspace_bytes, void* stream,
                           const int64_t* kdev, const int64_t* pdev, bool* one_launch) {
  Problem p;
  int rc = make_problem(cfg, out_features, in_features, k, &p);
  if (rc) return rc;
  p.kdev = kdev;
  p.pdev = pdev;
  const FwdLayout FL = fwd_layout(p);
  if (!forward_workspace || forward_workspace_bytes < FL.total)
    return set_err(GF_E_WORKSPACE, "forward workspace needs %zu bytes, got %zu", FL.total,
                   forward_workspace_bytes);
  uint8_t* fws = reinterpret_cast<uint8_t*>(forward_workspace);
  float* dg = reinterpret_cast<float*>(fws + FL.dgrad);  // [K][8]: d_amp, d_mu x2, d_chol_raw x3
  const bool direct = direct_one_launch(p, num_pairs, max_span) && k > 0;
  if (one_launch) *one_launch = direct;
  if (!direct) {
    rc = backward_reduce(cfg, out_features, in_features, k, grad_delta, row_coords, col_coords, mu, chol_raw,
                         tile_ptr, 1, gaussian_ids, 1, num_pairs, forward_workspace, workspace, workspace_bytes,
                         stream, kdev, pdev);
    if (rc) return rc;
    return backward_finish(cfg, out_features, in_features, k, chol_raw, amp, dg + 1, dg + 3, dg, forward_workspace,
                           workspace, workspace_bytes, stream, 8, kdev);
  }
  const BwdLayout L = bwd_layout(p);
  if (!workspace || workspace_bytes < L.total)
    return set_err(GF_E_WORKSPACE, "backward workspace needs %zu bytes, got %zu", L.total, workspace_bytes);
  if (num_pairs < 0) return set_err(GF_E_INVALID_ARGUMENT, "num_pairs must be non-negative");
  if (!grad_delta || !row_coords || !col_coords || !tile_ptr)
    return set_err(GF_E_INVALID_ARGUMENT, "grad_delta / coords / tile_ptr must not be NULL");
  if (num_pairs > 0 && !gaussian_ids) return set_err(GF_E_INVALID_ARGUMENT, "gaussian_ids must not be NULL");
  if (!mu || !chol_raw || !amp) return set_err(GF_E_INVALID_ARGUMENT, "mu / chol_raw / amp must not be NULL");
  if ((uint64_t)k * 8 >= (uint64_t)UINT32_MAX)
    return set_err(GF_E_INVALID_ARGUMENT, "k = %lld is too large for the direct gradients", (long long)k);
  hipStream_t st = reinterpret_cast<hipStream_t>(stream);
  const GaussEval* ev = reinterpret_cast<const GaussEval*>(fws + FL.eval);
  launch_bwd<int64_t, int64_t>(p, dim3((unsigned)((int64_t)p.R * p.C)), st, grad_delta, row_coords, col_coords,
                               mu, chol_raw, ev, tile_ptr, gaussian_ids, num_pairs,
                               reinterpret_cast<uint8_t*>(workspace), L,
                               reinterpret_cast<const int32_t*>(fws + FL.fill),
                               &reinterpret_cast<const WsHeader*>(fws)->heavy,
                               reinterpret_cast<const float4*>(fws + FL.dcoef), dg);
  GF_LAUNCH_CHECK("k_bwd");
  return GF_OK;
}

// The training backward: the one-launch kernel where the binning's facts allow it, its
// gradients then moved out of the slots (k_slots_out), otherwise gf_backward's reduction +
// finish.  The one-launch kernel reads what the mask-path binning left in forward_workspace (the
// constants, the chain-rule maps and the cleared slots), so it needs that workspace, int64 saved
// state, and the widest rectangle known (max_span >= 0).
int gf_backward_train(const gf_field_config* cfg, int64_t out_features, int64_t in_features, int64_t k,
                      const float* grad_delta, const float* row_coords, const float* col_coords, const float* mu,
                      const float* chol_raw, const float* amp, const void* tile_ptr, int32_t tile_ptr_is_int64,
                      const void* gaussian_ids, int32_t ids_is_int64, int64_t num_pairs, int64_t max_span,
                      float* d_mu, float* d_chol_raw, float* d_amp, void* forward_workspace, void* workspace,
                      size_t workspace_bytes, void* stream) {
  Problem p;
  int rc = make_problem(cfg, out_features, in_features, k, &p);
  if (rc) return rc;
  const bool direct = forward_workspace && tile_ptr_is_int64 == 1 && ids_is_int64 == 1 && max_span >= 0 &&
                      k > 0 && direct_one_launch(p, num_pairs, max_span);
  if (!direct)
    return gf_backward(cfg, out_features, in_features, k, grad_delta, row_coords, col_coords, mu, chol_raw, amp,
                       tile_ptr, tile_ptr_is_int64, gaussian_ids, ids_is_int64, num_pairs, d_mu, d_chol_raw, d_amp,
                       forward_workspace, workspace, workspace_bytes, stream);
  if (!d_mu || !d_chol_raw || !d_amp) return set_err(GF_E_INVALID_ARGUMENT, "d_mu / d_chol_raw / d_amp must not be NULL");
  const FwdLayout FL = fwd_layout(p);
  bool one = false;
  rc = backward_direct(cfg, out_features, in_features, k, grad_delta, row_coords, col_coords, mu, chol_raw, amp,
                       reinterpret_cast<const int64_t*>(tile_ptr), reinterpret_cast<const int64_t*>(gaussian_ids),
                       num_pairs, max_span, forward_workspace, FL.total, workspace, workspace_bytes, stream, nullptr,
                       nullptr, &one);
  if (rc) return rc;
  if (!one) return set_err(GF_E_INTERNAL, "gf_backward_train: the one-launch backward was not taken");
  hipStream_t st = reinterpret_cast<hipStream_t>(stream);
  float4* slots = reinterpret_cast<float4*>(reinterpret_cast<uint8_t*>(forward_workspace) + FL.dgrad);
  hipLaunchKernelGGL(k_slots_out, dim3((unsigned)((k + 255) / 256)), dim3(256), 0, st, slots, k, d_mu, d_chol_raw,
                     d_amp);
  GF_LAUNCH_CHECK("k_slots_out");
  return GF_OK;
}

// Capacity mode: the mask path at the capacity (every live K in [0, k_capacity] then takes the
// same kernels, grids and layouts).
static int check_kcap(const gf_field_config* cfg, int64_t out_features, int64_t in_features, int64_t k_capacity,
                      const int64_t* k_dev, Problem* p) {
  int rc = make_problem(cfg, out_features, in_features, k_capacity, p);
  if (rc) return rc;
  if (p->W == 0)
    return set_err(GF_E_INVALID_ARGUMENT,
                   "capacity mode takes 16x16 or 32x32 tiles with 1 <= k_capacity <= %lld (the mask path); "
                   "k_capacity = %lld", (long long)kMaskMaxK, (long long)k_capacity);
  if (!k_dev) return set_err(GF_E_INVALID_ARGUMENT, "k_dev must not be NULL");
  return GF_OK;
}

int gf_forward_kcap(const gf_field_config* cfg, int64_t out_features, int64_t in_features, int64_t k_capacity,
                    const int64_t* k_dev, const float* row_coords, const float* col_coords, const float* mu,
                    const float* chol_raw, const float* amp, int64_t* tile_ptr, int64_t* num_pairs_dev,
                    int64_t* gaussian_ids_sorted, int64_t ids_capacity, float* delta, void* workspace,
                    size_t workspace_bytes, void* stream) {
  Problem p;
  int rc = check_kcap(cfg, out_features, in_features, k_capacity, k_dev, &p);
  if (rc) return rc;
  rc = forward_bin(cfg, out_features, in_features, k_capacity, mu, chol_raw, amp, tile_ptr, num_pairs_dev, nullptr,
                   workspace, workspace_bytes, stream, false, k_dev);
  if (rc) return rc;
  return forward_render(cfg, out_features, in_features, k_capacity, row_coords, col_coords, tile_ptr,
                        gaussian_ids_sorted, ids_capacity, delta, workspace, workspace_bytes, stream, k_dev);
}

int gf_backward_direct_kcap(const gf_field_config* cfg, int64_t out_features, int64_t in_features,
                            int64_t k_capacity, const int64_t* k_dev, const float* grad_delta,
                            const float* row_coords, const float* col_coords, const float* mu,
                            const float* chol_raw, const float* amp, const int64_t* tile_ptr,
                            const int64_t* gaussian_ids, const int64_t* num_pairs_dev, int64_t ids_capacity,
                            void* forward_workspace, size_t forward_workspace_bytes, void* workspace,
                            size_t workspace_bytes, void* stream) {
  Problem p;
  int rc = check_kcap(cfg, out_features, in_features, k_capacity, k_dev, &p);
  if (rc) return rc;
  if (!num_pairs_dev) return set_err(GF_E_INVALID_ARGUMENT, "num_pairs_dev must not be NULL");
  return backward_direct(cfg, out_features, in_features, k_capacity, grad_delta, row_coords, col_coords, mu,
                         chol_raw, amp, tile_ptr, gaussian_ids, ids_capacity, -1, forward_workspace,
                         forward_workspace_bytes, workspace, workspace_bytes, stream, k_dev, num_pairs_dev);
}

// The one-pass kernel takes the fields gf_backward_direct runs in one launch, with 16x16 tiles and
// at least one Gaussian.
// (the fused kernel has no heavy-tile workgroups)
bool fused_one_pass(const Problem& p, int64_t pair_bound) {
  return p.K > 0 && p.tile_out == 16 && p.tile_in == 16 && direct_one_launch(p, pair_bound, -1) &&
         heavy_grid(p, pair_bound) == 0;
}

int gf_fwd_bwd_fused_supported(const gf_field_config* cfg, int64_t out_features, int64_t in_features, int64_t k,
                               int64_t ids_capacity, int64_t max_span) {
  Problem p;
  if (make_problem(cfg, out_features, in_features, k, &p)) return 0;
  return fused_one_pass(p, ids_capacity) && max_span < kDirectMaxSpan ? 1 : 0;
}

int gf_fwd_bwd_fused(const gf_field_config* cfg, int64_t out_features, int64_t in_features, int64_t k,
                     const float* row_coords, const float* col_coords, const float* mu, const float* chol_raw,
                     const float* amp, const float* grad_delta, int64_t* tile_ptr, int64_t* num_pairs_dev,
                     int64_t* gaussian_ids_sorted, int64_t ids_capacity, float* delta, void* forward_workspace,
                     size_t forward_workspace_bytes, void* stream) {
  Problem p;
  int rc = make_problem(cfg, out_features, in_features, k, &p);
  if (rc) return rc;
  if (!fused_one_pass(p, ids_capacity))
    return set_err(GF_E_INVALID_ARGUMENT,
                   "gf_fwd_bwd_fused takes 16x16 tiles on the mask path (1 <= k <= %lld) with fewer than 8192 "
                   "tiles, sparse and without heavy tiles (gf_fwd_bwd_fused_supported); run gf_forward + "
                   "gf_backward_direct for this field", (long long)kMaskMaxK);
  const FwdLayout FL = fwd_layout(p);
  if (!forward_workspace || forward_workspace_bytes < FL.total)
    return set_err(GF_E_WORKSPACE, "forward workspace needs %zu bytes, got %zu", FL.total, forward_workspace_bytes);
  if (!row_coords || !col_coords || !grad_delta || !delta || !amp)
    return set_err(GF_E_INVALID_ARGUMENT, "coords / grad_delta / delta / amp must not be NULL");
  if (ids_capacity < 0 || (ids_capacity > 0 && !gaussian_ids_sorted))
    return set_err(GF_E_INVALID_ARGUMENT, "gaussian_ids_sorted / ids_capacity invalid");
  if ((uint64_t)k * 8 >= (uint64_t)UINT32_MAX)
    return set_err(GF_E_INVALID_ARGUMENT, "k = %lld is too large for the direct gradients", (long long)k);
  // Fields within the row binning's limits (rows_fit) bin their tile rows in the fused kernel,
  // those of up to 256 Gaussians included (cfg1 11.0 -> 8.3 us, cfg2 13.0 -> 10.4 us against
  // k_bin_tiles' masks); the others take k_bin_tiles' masks.
  const bool rows = rows_fit(p);
  rc = forward_bin(cfg, out_features, in_features, k, mu, chol_raw, amp, tile_ptr, num_pairs_dev, nullptr,
                   forward_workspace, forward_workspace_bytes, stream, !rows);
  if (rc) return rc;
  hipStream_t st = reinterpret_cast<hipStream_t>(stream);
  uint8_t* fws = reinterpret_cast<uint8_t*>(forward_workspace);
  p.heavy = 0;
  const dim3 grid(rows ? (unsigned)((int64_t)p.R * ((p.C + kRowsThreads / 64 - 1) / (kRowsThreads / 64)))
                       : (unsigned)quad_grid(p));
  auto kern = rows ? (p.mask_clamp ? k_fused16<true, true> : k_fused16<false, true>)
                   : (p.mask_clamp ? k_fused16<true, false> : k_fused16<false, false>);
  hipLaunchKernelGGL(kern, grid, dim3(rows ? kRowsThreads : kTileThreads), 0, st, p, grad_delta, row_coords, col_coords,
                     reinterpret_cast<const GaussEval*>(fws + FL.eval), tile_ptr, gaussian_ids_sorted, ids_capacity,
                     delta, fws, reinterpret_cast<const uint32_t*>(fws + FL.rowmask),
                     reinterpret_cast<const uint32_t*>(fws + FL.colmask), reinterpret_cast<const float4*>(fws + FL.dcoef),
                     reinterpret_cast<float*>(fws + FL.dgrad), rows ? reinterpret_cast<const int4*>(fws + FL.rect) : nullptr,
                     rows ? tile_ptr : nullptr);
  GF_LAUNCH_CHECK("k_fused16");
  return GF_OK;
}

// ------------------------------------------------------------------------------------------
// Batched fields.

int gf_batch_plan(const gf_field_config* cfg, const gf_layer* layers, int32_t n_layers, void* plan,
                  size_t plan_bytes, gf_batch_info* info, void* stream) {
  if (!cfg || !info || n_layers < 0 || (n_layers > 0 && !layers))
    return set_err(GF_E_INVALID_ARGUMENT, "cfg / layers / info invalid");
  const bool t32 = cfg->tile_out == 32 && cfg->tile_in == 32;
  if (!(cfg->tile_out == 16 && cfg->tile_in == 16) && !t32)
    return set_err(GF_E_INVALID_ARGUMENT, "batched fields need 16x16 or 32x32 tiles (got %lldx%lld)",
                   (long long)cfg->tile_out, (long long)cfg->tile_in);
  const size_t n = (size_t)n_layers;
  BatchHeader h{};
  std::vector<BatchLayer> ls(n);
  int64_t tile_blocks = 0, emit_blocks = 0, finish_blocks = 0, render_blocks = 0;
  bool backward_buffers = true, grads_set = true, tile_render = false;
  for (size_t i = 0; i < n; ++i) {
    const gf_layer& in = layers[i];
    BatchLayer& ly = ls[i];
    int rc = make_problem(cfg, in.out_features, in.in_features, in.k, &ly.p);
    if (rc) {
      char why[sizeof(g_err)];
      std::snprintf(why, sizeof(why), "%s", g_err);
      return set_err(rc, "layer %zu: %s", i, why);
    }
    if (in.mu_tanh != 0 && in.mu_tanh != 1) return set_err(GF_E_INVALID_ARGUMENT, "layer %zu: mu_tanh must be 0 or 1", i);
    ly.p.mu_tanh = in.mu_tanh;
    const int64_t K = in.k;
    if (in.k_capacity < 0) return set_err(GF_E_INVALID_ARGUMENT, "layer %zu: k_capacity < 0", i);
    // Grids for the capacity: a layer on the emission path at any k <= kc keeps its emit blocks.
    const int64_t kc = std::max<int64_t>(K, in.k_capacity);
    Problem pc;
    rc = make_problem(cfg, in.out_features, in.in_features, kc, &pc);
    if (rc) return set_err(rc, "layer %zu: k_capacity %lld invalid", i, (long long)kc);
    if (t32 && !quad_render(ly.p))
      return set_err(GF_E_INVALID_ARGUMENT,
                     "layer %zu: batched 32x32 tiles need the mask path (1 <= k <= %lld, tile columns within LDS)",
                     i, (long long)kMaskMaxK);
    ly.fl = fwd_layout(ly.p);
    ly.bl = bwd_layout(ly.p);
    if (!in.forward_workspace || in.forward_workspace_bytes < ly.fl.total)
      return set_err(GF_E_WORKSPACE, "layer %zu: forward workspace needs %zu bytes", i, ly.fl.total);
    if (!in.row_coords || !in.col_coords || !in.tile_ptr || !in.num_pairs)
      return set_err(GF_E_INVALID_ARGUMENT, "layer %zu: coords / tile_ptr / num_pairs must not be NULL", i);
    if (!in.delta && !in.merged_weight)
      return set_err(GF_E_INVALID_ARGUMENT, "layer %zu: delta must not be NULL without a merged_weight", i);
    if (in.merged_weight && !in.base_weight)
      return set_err(GF_E_INVALID_ARGUMENT, "layer %zu: merged_weight needs base_weight", i);
    if (in.merged_weight && !(std::isfinite(in.delta_scale)))
      return set_err(GF_E_INVALID_ARGUMENT, "layer %zu: delta_scale must be finite", i);
    if (K > 0 && (!in.mu || !in.chol_raw || !in.amp))
      return set_err(GF_E_INVALID_ARGUMENT, "layer %zu: mu / chol_raw / amp must not be NULL", i);
    if (in.ids_capacity < 0 || (in.ids_capacity > 0 && !in.gaussian_ids))
      return set_err(GF_E_INVALID_ARGUMENT, "layer %zu: gaussian_ids / ids_capacity invalid", i);
    const bool bufs = in.backward_workspace && in.backward_workspace_bytes >= ly.bl.total &&
                      (K == 0 || (in.d_mu && in.d_chol_raw && in.d_amp));
    backward_buffers = backward_buffers && bufs;
    grads_set = grads_set && in.grad_delta;
    ly.row_coords = in.row_coords;
    ly.col_coords = in.col_coords;
    ly.mu = in.mu;
    ly.chol_raw = in.chol_raw;
    ly.amp = in.amp;
    ly.delta = in.delta;
    ly.tile_ptr = in.tile_ptr;
    ly.num_pairs = in.num_pairs;
    ly.ids = in.gaussian_ids;
    ly.capacity = in.ids_capacity;
    ly.fws = reinterpret_cast<uint8_t*>(in.forward_workspace);
    ly.bws = reinterpret_cast<uint8_t*>(in.backward_workspace);
    ly.d_mu = in.d_mu;
    ly.d_chol_raw = in.d_chol_raw;
    ly.d_amp = in.d_amp;
    ly.tile_block0 = tile_blocks;
    ly.emit_block0 = emit_blocks;
    ly.finish_block0 = finish_blocks;
    ly.render_block0 = render_blocks;
    tile_blocks += quad_grid(ly.p);
    // Tile pairs for 16x16 layers on the mask path at the capacity, hence at every 1 <= k <= kc
    // (each condition of the mask path bounds K from above; the grids must not change with k).
    // The others render tile by tile over the tile map: layers past the masks' K, and layers
    // narrower than a tile, whose tile make_problem clamps to the matrix (emission path).
    ly.pair_render = (!t32 && pc.W > 0) ? 1 : 0;
    ly.mo.base = in.merged_weight ? in.base_weight : nullptr;
    ly.mo.merged = in.merged_weight;
    ly.mo.scale = in.merged_weight ? in.delta_scale : 1.0f;
    ly.grad_scale = ly.mo.scale;
    if (ly.pair_render)
      render_blocks += ((int64_t)ly.p.R * ((ly.p.C + 1) / 2) + kTileThreads / 64 - 1) / (kTileThreads / 64);
    else
      tile_render = true;
    const int64_t per_emit_block = (kEmitThreads / 64) * (64 / kEmitLanesBatch);
    if (ly.p.W == 0 || pc.W == 0) emit_blocks += (kc + per_emit_block - 1) / per_emit_block;  // emission path
    finish_blocks += (kc * ly.p.S + kTileThreads - 1) / kTileThreads;
  }
  if (tile_blocks >= INT32_MAX || emit_blocks >= INT32_MAX || render_blocks >= INT32_MAX)
    return set_err(GF_E_INVALID_ARGUMENT, "batch too large for one launch");
  h = batch_header(n_layers, tile_blocks, emit_blocks, finish_blocks, render_blocks);
  const size_t need = (size_t)h.total;
  info->n_layers = n_layers;
  info->mask_clamp = (cfg->has_clamp_quad && cfg->clamp_quad < 80.0) ? 1 : 0;
  info->backward_buffers = backward_buffers ? 1 : 0;
  info->has_backward = backward_buffers && grads_set ? 1 : 0;
  info->tile_blocks = tile_blocks;
  info->emit_blocks = emit_blocks;
  info->finish_blocks = finish_blocks;
  info->render_blocks = render_blocks;
  info->tile_render = tile_render ? 1 : 0;
  info->reserved = 0;
  info->plan_bytes = need;
  if (!plan) return GF_OK;  // size query
  if (plan_bytes < need) return set_err(GF_E_WORKSPACE, "batch plan needs %zu bytes, got %zu", need, plan_bytes);
  std::vector<uint8_t> host(need, 0);
  std::memcpy(host.data(), &h, sizeof(h));
  if (n) std::memcpy(host.data() + h.layers_off, ls.data(), sizeof(BatchLayer) * n);
  int32_t* tm = reinterpret_cast<int32_t*>(host.data() + h.tile_map_off);
  int32_t* em = reinterpret_cast<int32_t*>(host.data() + h.emit_map_off);
  int32_t* fm = reinterpret_cast<int32_t*>(host.data() + h.finish_map_off);
  int32_t* rmap = reinterpret_cast<int32_t*>(host.data() + h.render_map_off);
  const float** gt = reinterpret_cast<const float**>(host.data() + h.grad_table_off);
  for (size_t i = 0; i < n; ++i) gt[i] = layers[i].grad_delta;
  for (size_t i = 0; i < n; ++i) {
    const int64_t te = i + 1 < n ? ls[i + 1].tile_block0 : tile_blocks;
    const int64_t ee = i + 1 < n ? ls[i + 1].emit_block0 : emit_blocks;
    const int64_t fe = i + 1 < n ? ls[i + 1].finish_block0 : finish_blocks;
    const int64_t re = i + 1 < n ? ls[i + 1].render_block0 : render_blocks;
    for (int64_t b = ls[i].tile_block0; b < te; ++b) tm[b] = (int32_t)i;
    for (int64_t b = ls[i].emit_block0; b < ee; ++b) em[b] = (int32_t)i;
    for (int64_t b = ls[i].finish_block0; b < fe; ++b) fm[b] = (int32_t)i;
    for (int64_t b = ls[i].render_block0; b < re; ++b) rmap[b] = (int32_t)i;
  }
  hipStream_t st = reinterpret_cast<hipStream_t>(stream);
  GF_HIP_CHECK(hipMemcpyAsync(plan, host.data(), need, hipMemcpyHostToDevice, st));
  GF_HIP_CHECK(hipStreamSynchronize(st));  // the host staging buffer goes out of scope
  return GF_OK;
}

int gf_batch_forward(const void* plan, const gf_batch_info* info, uint32_t phases, void* stream) {
  if (!plan || !info) return set_err(GF_E_INVALID_ARGUMENT, "plan / info must not be NULL");
  if (info->n_layers == 0) return GF_OK;
  hipStream_t st = reinterpret_cast<hipStream_t>(stream);
  const uint8_t* pl = reinterpret_cast<const uint8_t*>(plan);
  if (phases & GF_PHASE_BIN) {
    hipLaunchKernelGGL(k_bin_batch, dim3((unsigned)info->n_layers), dim3(kBinThreads), 0, st, pl);
    GF_LAUNCH_CHECK("k_bin_batch");
  }
  if ((phases & GF_PHASE_EMIT) && info->emit_blocks > 0) {
    hipLaunchKernelGGL(k_emit_batch, dim3((unsigned)info->emit_blocks), dim3(kEmitThreads), 0, st, pl);
    GF_LAUNCH_CHECK("k_emit_batch");
  }
  if (phases & GF_PHASE_RENDER) {
    if (info->render_blocks > 0) {
      hipLaunchKernelGGL(k_render16x2_batch, dim3((unsigned)info->render_blocks), dim3(kTileThreads), 0, st, pl);
      GF_LAUNCH_CHECK("k_render16x2_batch");
    }
    if (info->tile_render) {
      hipLaunchKernelGGL(k_render16_batch, dim3((unsigned)info->tile_blocks), dim3(kTileThreads), 0, st, pl);
      GF_LAUNCH_CHECK("k_render16_batch");
    }
  }
  return GF_OK;
}

int gf_batch_set_grads(void* plan, gf_batch_info* info, const float* const* grad_delta, void* stream) {
  if (!plan || !info || (info->n_layers > 0 && !grad_delta))
    return set_err(GF_E_INVALID_ARGUMENT, "plan / info / grad_delta must not be NULL");
  bool all = true;
  for (int32_t i = 0; i < info->n_layers; ++i) all = all && grad_delta[i];
  if (!all) return set_err(GF_E_INVALID_ARGUMENT, "every layer needs a dL/d(delta) pointer");
  hipStream_t st = reinterpret_cast<hipStream_t>(stream);
  uint8_t* pl = reinterpret_cast<uint8_t*>(plan);
  for (int32_t b = 0; b < info->n_layers; b += kPtrChunk) {
    PtrChunk c{};
    const int32_t cnt = std::min<int32_t>(kPtrChunk, info->n_layers - b);
    for (int32_t i = 0; i < cnt; ++i) c.p[i] = grad_delta[b + i];
    hipLaunchKernelGGL(k_batch_set_grads, dim3(1), dim3(kPtrChunk), 0, st, pl, c, b, cnt);
    GF_LAUNCH_CHECK("k_batch_set_grads");
  }
  info->has_backward = info->backward_buffers;
  return GF_OK;
}

int gf_batch_read(void* plan, const gf_batch_info* info, int32_t clear, uint32_t* status_host,
                  int64_t* pairs_host, double* delta_norm_host, void* stream) {
  if (!plan || !info) return set_err(GF_E_INVALID_ARGUMENT, "plan / info must not be NULL");
  const int32_t n = info->n_layers;
  if (n == 0) return GF_OK;
  hipStream_t st = reinterpret_cast<hipStream_t>(stream);
  uint8_t* pl = reinterpret_cast<uint8_t*>(plan);
  hipLaunchKernelGGL(k_batch_read, dim3((unsigned)n), dim3(256), 0, st, pl, clear);
  GF_LAUNCH_CHECK("k_batch_read");
  const BatchHeader h = batch_header(n, info->tile_blocks, info->emit_blocks, info->finish_blocks, info->render_blocks);
  std::vector<BatchReadback> rb((size_t)n);
  GF_HIP_CHECK(hipMemcpyAsync(rb.data(), pl + h.readback_off, sizeof(BatchReadback) * (size_t)n,
                              hipMemcpyDeviceToHost, st));
  GF_HIP_CHECK(hipStreamSynchronize(st));
  for (int32_t i = 0; i < n; ++i) {
    if (status_host) status_host[i] = rb[(size_t)i].status;
    if (pairs_host) pairs_host[i] = rb[(size_t)i].pairs;
    if (delta_norm_host) delta_norm_host[i] = std::sqrt(rb[(size_t)i].delta_sumsq);
  }
  return GF_OK;
}

int gf_batch_backward(const void* plan, const gf_batch_info* info, uint32_t phases, void* stream) {
  if (!plan || !info) return set_err(GF_E_INVALID_ARGUMENT, "plan / info must not be NULL");
  if (!info->has_backward)
    return set_err(GF_E_INVALID_ARGUMENT,
                   "the batch plan has no backward buffers or no dL/d(delta) pointers (gf_batch_set_grads)");
  if (info->n_layers == 0) return GF_OK;
  hipStream_t st = reinterpret_cast<hipStream_t>(stream);
  const uint8_t* pl = reinterpret_cast<const uint8_t*>(plan);
  if (phases & GF_PHASE_REDUCE) {
    if (info->mask_clamp)
      hipLaunchKernelGGL(k_bwd16_batch<true>, dim3((unsigned)info->tile_blocks), dim3(kTileThreads), 0, st, pl);
    else
      hipLaunchKernelGGL(k_bwd16_batch<false>, dim3((unsigned)info->tile_blocks), dim3(kTileThreads), 0, st, pl);
    GF_LAUNCH_CHECK("k_bwd16_batch");
  }
  if ((phases & GF_PHASE_FINISH) && info->finish_blocks > 0) {
    hipLaunchKernelGGL(k_finish_batch, dim3((unsigned)info->finish_blocks), dim3(kTileThreads), 0, st, pl);
    GF_LAUNCH_CHECK("k_finish_batch");
  }
  return GF_OK;
}

int gf_backward_noalloc(const gf_field_config* cfg, int64_t out_features, int64_t in_features, int64_t k,
                        const float* grad_delta, const float* row_coords, const float* col_coords,
                        const float* mu, const float* chol_raw, const float* amp, const void* tile_ptr,
                        int32_t tile_ptr_is_int64, const void* gaussian_ids, int32_t ids_is_int64,
                        int64_t num_pairs, float* d_mu, float* d_chol_raw, float* d_amp, uint32_t* status_dev,
                        void* stream) {
  Problem p;
  int rc = make_problem(cfg, out_features, in_features, k, &p);
  if (rc) return rc;
  const BwdLayout L = bwd_layout(p);
  if (L.total > kNoAllocScratchBytes)
    return set_err(GF_E_WORKSPACE,
                   "gf_backward_noalloc: this field needs %zu bytes of backward workspace; the static scratch "
                   "holds %zu (K <= %lld for %d accumulator stripes); use gf_backward with a workspace",
                   L.total, kNoAllocScratchBytes,
                   (long long)((kNoAllocScratchBytes - sizeof(WsHeader)) / (32 * (size_t)p.S)), (int)p.S);
  if (k > 0 && !amp) return set_err(GF_E_INVALID_ARGUMENT, "amp must not be NULL");
  void* ws = nullptr;
  rc = scratch_for_current_device(&ws);
  if (rc) return rc;
  hipStream_t st = reinterpret_cast<hipStream_t>(stream);
  // the header (status word) and this call's accumulator slots start at zero
  const int64_t words = (int64_t)(L.total / 16);
  hipLaunchKernelGGL(k_fill_zero, dim3((unsigned)std::min<int64_t>((words + 255) / 256, 1024)), dim3(256), 0, st,
                     reinterpret_cast<uint4*>(ws), words);
  GF_LAUNCH_CHECK("k_fill_zero");
  rc = gf_backward(cfg, out_features, in_features, k, grad_delta, row_coords, col_coords, mu, chol_raw, amp,
                   tile_ptr, tile_ptr_is_int64, gaussian_ids, ids_is_int64, num_pairs, d_mu, d_chol_raw, d_amp,
                   nullptr, ws, L.total, stream);
  if (rc) return rc;
  if (status_dev) {
    hipLaunchKernelGGL(k_copy_status, dim3(1), dim3(64), 0, st, reinterpret_cast<const uint32_t*>(ws), status_dev);
    GF_LAUNCH_CHECK("k_copy_status");
  }
  return GF_OK;
}

int gf_read_bin_info(const void* forward_workspace, gf_bin_info* info, void* stream) {
  if (!forward_workspace || !info)
    return set_err(GF_E_INVALID_ARGUMENT, "forward_workspace / info must not be NULL");
  hipStream_t st = reinterpret_cast<hipStream_t>(stream);
  void* pinned = nullptr;
  int rc = pinned_readback(&pinned);
  if (rc) return rc;
  GF_HIP_CHECK(hipMemcpyAsync(pinned, forward_workspace, offsetof(WsHeader, max_span) + sizeof(int64_t),
                              hipMemcpyDeviceToHost, st));
  GF_HIP_CHECK(hipStreamSynchronize(st));
  const WsHeader* h = reinterpret_cast<const WsHeader*>(pinned);
  info->num_pairs = h->pairs;
  info->max_span = h->max_span;
  return GF_OK;
}

int gf_read_status(void* workspace, int32_t clear, uint32_t* status_host, void* stream) {
  if (!workspace || !status_host) return set_err(GF_E_INVALID_ARGUMENT, "workspace / status_host must not be NULL");
  hipStream_t st = reinterpret_cast<hipStream_t>(stream);
  WsHeader* hdr = reinterpret_cast<WsHeader*>(workspace);
  void* pinned = nullptr;
  int rc = pinned_readback(&pinned);
  if (rc) return rc;
  GF_HIP_CHECK(hipMemcpyAsync(pinned, &hdr->status, sizeof(uint32_t), hipMemcpyDeviceToHost, st));
  GF_HIP_CHECK(hipStreamSynchronize(st));
  const uint32_t v = *reinterpret_cast<const uint32_t*>(pinned);
  *status_host = v;
  if (clear && v != 0u) {  // a clean word (the usual case) needs no clearing launch
    hipLaunchKernelGGL(k_clear_status, dim3(1), dim3(64), 0, st, &hdr->status);
    GF_LAUNCH_CHECK("k_clear_status");
  }
  return GF_OK;
}

int gf_selftest_softplus(uint64_t* checksum_host, void* stream) {
  if (!checksum_host) return set_err(GF_E_INVALID_ARGUMENT, "checksum_host must not be NULL");
  hipStream_t st = reinterpret_cast<hipStream_t>(stream);
  unsigned long long* d = nullptr;
  GF_HIP_CHECK(hipMalloc(&d, sizeof(unsigned long long)));
  const unsigned long long zero = 0;
  hipError_t e = hipMemcpyAsync(d, &zero, sizeof(zero), hipMemcpyHostToDevice, st);
  if (e == hipSuccess) {
    hipLaunchKernelGGL(k_selftest_softplus, dim3(8192), dim3(256), 0, st, d);
    e = hipGetLastError();
  }
  unsigned long long h = 0;
  if (e == hipSuccess) e = hipMemcpyAsync(&h, d, sizeof(h), hipMemcpyDeviceToHost, st);
  if (e == hipSuccess) e = hipStreamSynchronize(st);
  (void)hipFree(d);
  if (e != hipSuccess) return set_err(GF_E_HIP, "softplus self-test failed: %s", hipGetErrorString(e));
  *checksum_host = (uint64_t)h;
  return GF_OK;
}

}  // extern "C"
