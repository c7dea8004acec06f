// gaussfield.hip - gfx950 kernels and C ABI of libgaussfield.so.
//
// Forward (reference forward.cu:372-569):
//   k_bin     one workgroup per problem: per-Gaussian geometry, sigma-box tile rectangles
//             (bit-exact with the CPU path), exclusive scan of tiles touched per Gaussian
//             ("point offsets"), per-tile Gaussian counts from row-wise difference arrays in
//             LDS, exclusive scan of the counts -> tile_ptr.  No global atomics, no host sync.
//   k_emit    one thread per (gaussian, tile) pair: finds its Gaussian by binary search of the
//             point offsets, claims a slot in its tile's range (a counting sort on the tile key:
//             one 64-bit atomic per pair on a per-tile cursor) and stores the gaussian id.
//   k_render  one workgroup per tile: puts the tile's ids in canonical (ascending gid) order in
//             LDS and writes them back, stages the tile's Gaussians in LDS and evaluates every
//             pixel of the tile, writing delta-W with row-coalesced stores.  Empty tiles get 0.
// Backward (reference backward.cu:541-716), one kernel:
//   k_bwd_tiles one workgroup per tile: geometry of the tile's Gaussians in LDS, six
//               per-Gaussian pixel sums reduced across the workgroup, one atomic per
//               (Gaussian, tile, sum); the last workgroup to finish applies the chain rule to
//               (mu, chol_raw, amp) and clears the accumulators for the next call.
#include <hip/hip_runtime.h>

#include <algorithm>
#include <cstdarg>
#include <cstdint>
#include <cstdio>
#include <cstring>

#include "../../include/gaussfield.h"
#include "geometry.h"

#define GF_VERSION "gaussfield-mi355x 0.1.0"

namespace {

constexpr int kBinThreads = 1024;
constexpr int kTileThreads = 256;
constexpr int kEmitThreads = 256;
constexpr int kLdsDiffWords = 12288;   // 48 KiB row-difference band in k_bin
constexpr int kSortLdsKeys = 2048;     // segments up to this length are ordered in LDS
constexpr int kBitmapMaxK = 131072;    // longer segments use a K-bit bitmap when K fits
constexpr float kLog2e = 1.4426950408889634f;

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
// Problem description (passed by value as a kernel argument).
struct Problem {
  int64_t M, N, K;
  int64_t tile_out, tile_in;
  int64_t R, C;  // tile rows / cols
  float sigma;
  float clamp_quad;
  int32_t normalize;
  int32_t has_clamp;
};

// Render geometry of one Gaussian in fp32 (32 bytes).
struct __align__(16) GeomF {
  float mu0, mu1, i00, i01, i11, norm, det, pad;
};

// Header of every workspace.
struct WsHeader {
  uint32_t status;
  uint32_t ticket;
  uint32_t pad[62];
};
static_assert(sizeof(WsHeader) == 256, "workspace header must be 256 bytes");

size_t align256(size_t x) { return (x + 255) & ~size_t(255); }

struct FwdLayout {
  size_t geo, rect, offs, cursor, total;
};
FwdLayout fwd_layout(int64_t K, int64_t T) {
  FwdLayout L;
  size_t o = sizeof(WsHeader);
  L.geo = o;
  o = align256(o + sizeof(GeomF) * (size_t)K);
  L.rect = o;
  o = align256(o + sizeof(int4) * (size_t)K);
  L.offs = o;
  o = align256(o + sizeof(int64_t) * (size_t)(K + 1));
  L.cursor = o;
  o = align256(o + sizeof(int64_t) * (size_t)T);
  L.total = o;
  return L;
}

// Backward workspace: header + eight fp32 accumulators per Gaussian.  It must be zero before
// the first backward; every backward leaves it zero again (the last workgroup clears what it
// consumed), so a workspace kept across calls is zeroed once.
struct BwdLayout {
  size_t acc, total;
};
BwdLayout bwd_layout(int64_t K) {
  BwdLayout L;
  size_t o = sizeof(WsHeader);
  L.acc = o;
  o = align256(o + sizeof(float) * 8 * (size_t)K);
  L.total = o;
  return L;
}

__device__ inline void set_status(uint32_t* status, uint32_t bit) { atomicOr(status, bit); }

// Render geometry + bit-exact rectangle of Gaussian g.
__device__ inline void gaussian_geometry(const Problem& p, const float* __restrict__ mu,
                                         const float* __restrict__ chol_raw, int64_t g, GeomF* geo,
                                         GfRect* rect) {
  const float mu0 = mu[2 * g + 0], mu1 = mu[2 * g + 1];
  const GfChol L = gf_activate_cholesky(chol_raw[3 * g + 0], chol_raw[3 * g + 1], chol_raw[3 * g + 2]);
  const GfCov cov = gf_cov_from_chol(L);
  if (rect) *rect = gf_tile_rect(mu0, mu1, cov, p.M, p.N, p.tile_out, p.tile_in, p.R, p.C, p.sigma);
  const GfRenderGeom rg = gf_render_geom(cov, p.normalize);
  geo->mu0 = mu0;
  geo->mu1 = mu1;
  geo->i00 = (float)rg.i00;
  geo->i01 = (float)rg.i01;
  geo->i11 = (float)rg.i11;
  geo->norm = rg.norm;
  geo->det = rg.det_f;
  geo->pad = 0.0f;
}

// ------------------------------------------------------------------------------------------
// Workgroup scans.

__device__ inline int64_t wave_inclusive_scan(int64_t x) {
  const int lane = threadIdx.x & 63;
#pragma unroll
  for (int o = 1; o < 64; o <<= 1) {
    const int64_t y = __shfl_up(x, o, 64);
    if (lane >= o) x += y;
  }
  return x;
}

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

__global__ __launch_bounds__(kBinThreads) void k_bin(Problem p, const float* __restrict__ mu,
                                                     const float* __restrict__ chol_raw,
                                                     int64_t* __restrict__ tile_ptr,
                                                     int64_t* __restrict__ num_pairs, uint8_t* ws,
                                                     FwdLayout L) {
  __shared__ int32_t diff[kLdsDiffWords];
  __shared__ int64_t scan_lds[kBinThreads / 64 + 1];
  WsHeader* hdr = reinterpret_cast<WsHeader*>(ws);
  GeomF* geo = reinterpret_cast<GeomF*>(ws + L.geo);
  int4* rect = reinterpret_cast<int4*>(ws + L.rect);
  int64_t* offs = reinterpret_cast<int64_t*>(ws + L.offs);
  int64_t* cursor = reinterpret_cast<int64_t*>(ws + L.cursor);
  const int64_t K = p.K, T = p.R * p.C;
  if (threadIdx.x == 0) {
    hdr->status = 0u;
    hdr->ticket = 0u;
  }

  // A: geometry, rectangles, tiles touched.
  for (int64_t g = threadIdx.x; g < K; g += kBinThreads) {
    GeomF gf;
    GfRect r;
    gaussian_geometry(p, mu, chol_raw, g, &gf, &r);
    geo[g] = gf;
    rect[g] = make_int4((int)r.r0, (int)r.r1, (int)r.c0, (int)r.c1);
    offs[g] = (r.r1 - r.r0 + 1) * (r.c1 - r.c0 + 1);
  }
  __syncthreads();

  // B: point offsets (exclusive scan of tiles touched); offs[K] = P.
  const int64_t P = block_scan_runs<kBinThreads>(offs, K, scan_lds);
  if (threadIdx.x == 0) offs[K] = P;

  // C: per-tile counts, band by band.  A band covers rows [b0, b0+nb) and columns
  // [cb0, cb0+W) of the tile grid; each covered row of each rectangle adds +1 at its first
  // column and -1 after its last, and a row scan turns the differences into counts.
  const int64_t W = p.C < kLdsDiffWords ? p.C : kLdsDiffWords;
  const int64_t band_rows = kLdsDiffWords / W;
  for (int64_t cb0 = 0; cb0 < p.C; cb0 += W) {
    const int64_t wb = (p.C - cb0) < W ? (p.C - cb0) : W;
    for (int64_t b0 = 0; b0 < p.R; b0 += band_rows) {
      const int64_t nb = (p.R - b0) < band_rows ? (p.R - b0) : band_rows;
      for (int64_t i = threadIdx.x; i < nb * wb; i += kBinThreads) diff[i] = 0;
      __syncthreads();
      for (int64_t g = threadIdx.x; g < K; g += kBinThreads) {
        const int4 r = rect[g];
        const int64_t rlo = r.x > b0 ? r.x : b0;
        const int64_t rhi = r.y < b0 + nb - 1 ? r.y : b0 + nb - 1;
        const int64_t clo = r.z > cb0 ? r.z : cb0;
        const int64_t chi = r.w < cb0 + wb - 1 ? r.w : cb0 + wb - 1;
        if (rlo > rhi || clo > chi) continue;
        for (int64_t row = rlo; row <= rhi; ++row) {
          int32_t* d = diff + (row - b0) * wb;
          atomicAdd(d + (clo - cb0), 1);
          if (chi + 1 < cb0 + wb) atomicAdd(d + (chi + 1 - cb0), -1);
        }
      }
      __syncthreads();
      // Row scans: one wave per row.
      const int lane = threadIdx.x & 63, wid = threadIdx.x >> 6;
      for (int64_t row = wid; row < nb; row += kBinThreads / 64) {
        int64_t carry = 0;
        for (int64_t j0 = 0; j0 < wb; j0 += 64) {
          const int64_t j = j0 + lane;
          const int64_t v = j < wb ? diff[row * wb + j] : 0;
          const int64_t inc = wave_inclusive_scan(v) + carry;
          if (j < wb) tile_ptr[(b0 + row) * p.C + cb0 + j] = inc;  // count of tile
          carry = __shfl(inc, 63, 64);
        }
      }
      __syncthreads();
    }
  }

  // D: tile_ptr = exclusive scan of counts; cursors start at each tile's first slot.
  const int64_t Pc = block_scan_runs<kBinThreads>(tile_ptr, T, scan_lds);
  for (int64_t t = threadIdx.x; t < T; t += kBinThreads) cursor[t] = tile_ptr[t];
  if (threadIdx.x == 0) {
    tile_ptr[T] = Pc;
    *num_pairs = P;
    if (Pc != P) hdr->status |= GF_STATUS_COUNT_MISMATCH;
  }
}

// ------------------------------------------------------------------------------------------
// k_emit: one thread per pair (grid-stride).

__global__ __launch_bounds__(kEmitThreads) void k_emit(Problem p, uint8_t* ws, FwdLayout L,
                                                       int64_t* __restrict__ ids, int64_t capacity) {
  WsHeader* hdr = reinterpret_cast<WsHeader*>(ws);
  const int4* __restrict__ rect = reinterpret_cast<const int4*>(ws + L.rect);
  const int64_t* __restrict__ offs = reinterpret_cast<const int64_t*>(ws + L.offs);
  unsigned long long* cursor = reinterpret_cast<unsigned long long*>(ws + L.cursor);
  const int64_t K = p.K;
  const int64_t P = offs[K];
  const int64_t stride = (int64_t)gridDim.x * blockDim.x;
  for (int64_t pi = (int64_t)blockIdx.x * blockDim.x + threadIdx.x; pi < P; pi += stride) {
    // Largest g with offs[g] <= pi (offs strictly increasing: every Gaussian touches >= 1 tile).
    int64_t lo = 0, hi = K - 1;
    while (lo < hi) {
      const int64_t mid = (lo + hi + 1) >> 1;
      if (offs[mid] <= pi) lo = mid; else hi = mid - 1;
    }
    const int64_t g = lo;
    const int64_t local = pi - offs[g];
    const int4 r = rect[g];
    const int64_t w = (int64_t)(r.w - r.z + 1);
    const int64_t tr = r.x + local / w;
    const int64_t tc = r.z + local % w;
    const int64_t t = tr * p.C + tc;
    const unsigned long long pos = atomicAdd(cursor + t, 1ull);
    if ((int64_t)pos < capacity) ids[pos] = g;
    else set_status(&hdr->status, GF_STATUS_CAPACITY);
  }
}

// ------------------------------------------------------------------------------------------
// Canonical (ascending) order of a tile's id segment.

// Ascending bitonic sort by one workgroup, "flip" form: the first step of every merge stage
// pairs i with its mirror i ^ (k-1), later steps pair i with i ^ j, and the smaller key always
// goes to the lower index.  Indices >= n behave as +infinity and are never touched, so no
// padding is stored.
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

// Orders seg[0..n) ascending.  lds_words: LDS scratch (>= max(kSortLdsKeys, K/32) int32).
__device__ void sort_segment(int64_t* seg, int64_t n, int64_t K, int32_t* lds, int64_t* lds_small,
                             uint32_t* status) {
  if (n <= 1) return;
  if (n <= kSortLdsKeys) {
    for (int64_t i = threadIdx.x; i < n; i += blockDim.x) lds[i] = (int32_t)seg[i];
    __syncthreads();
    bitonic_sort_ascending<int32_t>(lds, n);
    for (int64_t i = threadIdx.x; i < n; i += blockDim.x) seg[i] = lds[i];
    __syncthreads();
    return;
  }
  if (K <= kBitmapMaxK) {
    // Distinct ids in [0, K): set bits, scan popcounts, expand in order.
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
    // Each thread owns a contiguous run of words.
    const int64_t per = (words + blockDim.x - 1) / blockDim.x;
    const int64_t wb = (int64_t)threadIdx.x * per;
    const int64_t we = wb + per < words ? wb + per : words;
    int64_t cnt = 0;
    for (int64_t w = wb; w < we; ++w) cnt += __popc(bits[w]);
    int64_t total;
    int64_t pos = block_exclusive_scan<kTileThreads>(cnt, &total, lds_small);
    if (total != n) {
      if (threadIdx.x == 0) set_status(status, GF_STATUS_COUNT_MISMATCH);
    }
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

// ------------------------------------------------------------------------------------------
// k_render: one workgroup per tile.

struct __align__(16) GaussLds {
  float mu0, mu1, i00, i01, i11, w;  // w = amp * norm
  float pad0, pad1;
};

__global__ __launch_bounds__(kTileThreads) void k_render(
    Problem p, const float* __restrict__ row_coords, const float* __restrict__ col_coords,
    const float* __restrict__ amp, const int64_t* __restrict__ tile_ptr, int64_t* ids,
    int64_t capacity, float* __restrict__ delta, uint8_t* ws, FwdLayout L) {
  __shared__ int32_t sort_lds[(kSortLdsKeys > kBitmapMaxK / 32) ? kSortLdsKeys : kBitmapMaxK / 32];
  __shared__ int64_t small_lds[kTileThreads / 64 + 1];
  __shared__ GaussLds gl[kTileThreads];
  WsHeader* hdr = reinterpret_cast<WsHeader*>(ws);
  const GeomF* __restrict__ geo = reinterpret_cast<const GeomF*>(ws + L.geo);
  const int64_t t = blockIdx.x;
  const int64_t tr = t / p.C, tc = t % p.C;
  int64_t s = tile_ptr[t], e = tile_ptr[t + 1];
  if (e > capacity) e = capacity;
  if (s > e) s = e;
  const int64_t n = e - s;
  int64_t* seg = ids + s;
  sort_segment(seg, n, p.K, sort_lds, small_lds, &hdr->status);

  const int64_t r0 = tr * p.tile_out, c0 = tc * p.tile_in;
  const int64_t r1 = (r0 + p.tile_out) < p.M ? (r0 + p.tile_out) : p.M;
  const int64_t c1 = (c0 + p.tile_in) < p.N ? (c0 + p.tile_in) : p.N;
  const int64_t w = c1 - c0;
  const int64_t npx = (r1 - r0) * w;
  for (int64_t px0 = 0; px0 < npx; px0 += kTileThreads) {
    const int64_t px = px0 + threadIdx.x;
    const bool have = px < npx;
    const int64_t r = r0 + (have ? px / w : 0);
    const int64_t c = c0 + (have ? px % w : 0);
    const float x = row_coords[r], y = col_coords[c];
    float acc = 0.0f;
    for (int64_t j0 = 0; j0 < n; j0 += kTileThreads) {
      const int64_t nj = (n - j0) < kTileThreads ? (n - j0) : kTileThreads;
      __syncthreads();
      if (threadIdx.x < nj) {
        const int64_t g = seg[j0 + threadIdx.x];
        GaussLds v;
        if (g >= 0 && g < p.K) {
          const GeomF q = geo[g];
          v.mu0 = q.mu0;
          v.mu1 = q.mu1;
          v.i00 = q.i00;
          v.i01 = q.i01;
          v.i11 = q.i11;
          v.w = amp[g] * q.norm;
        } else {  // only reachable after an internal count mismatch (status already flagged)
          v.mu0 = v.mu1 = v.i00 = v.i01 = v.i11 = v.w = 0.0f;
          set_status(&hdr->status, GF_STATUS_COUNT_MISMATCH);
        }
        v.pad0 = v.pad1 = 0.0f;
        gl[threadIdx.x] = v;
      }
      __syncthreads();
      for (int j = 0; j < (int)nj; ++j) {
        const GaussLds v = gl[j];
        const float dx = x - v.mu0, dy = y - v.mu1;
        float q = (dx * v.i00 + dy * v.i01) * dx + (dx * v.i01 + dy * v.i11) * dy;
        if (p.has_clamp) q = fminf(fmaxf(q, 0.0f), p.clamp_quad);
        acc += v.w * expf(-0.5f * q);
      }
    }
    if (have) delta[r * p.N + c] = acc;
  }
}

// ------------------------------------------------------------------------------------------
// Backward.

__device__ inline float wave_sum(float v) {
#pragma unroll
  for (int o = 32; o > 0; o >>= 1) v += __shfl_xor(v, o, 64);
  return v;
}

template <typename Idx>
__device__ inline int64_t load_idx(const void* p, int64_t i) {
  return (int64_t)reinterpret_cast<const Idx*>(p)[i];
}

// Chain rule from the six pixel sums of Gaussian g to (d_mu, d_chol_raw, d_amp), in double.
//   S0 = sum g e, S1 = sum w dx, S2 = sum w dy, S3 = sum w dx^2, S4 = sum w dx dy, S5 = sum w dy^2
// with e = exp(-q/2) (clamped q), w = g e [q inside the clamp range].  Derivation:
//   d_amp = norm S0;  d_mu = amp norm A (S1, S2);  dL/dA = -amp norm / 2 [[S3,S4],[S4,S5]];
//   dL/ddet = amp S0 (-norm / (2 det)) if normalize and sqrt(det) >= eps;
//   dL/dcov = -A (dL/dA) A + dL/ddet det A;  dL/dL = (G + G^T) L;  softplus' on the diagonal.
__device__ void chain_one(const Problem& p, const float* __restrict__ mu, const float* __restrict__ chol_raw,
                          const float* __restrict__ amp, const float* acc8, int64_t g,
                          float* __restrict__ d_mu, float* __restrict__ d_chol_raw,
                          float* __restrict__ d_amp) {
  const float raw11 = chol_raw[3 * g + 0], raw21 = chol_raw[3 * g + 1], raw22 = chol_raw[3 * g + 2];
  const GfChol Lc = gf_activate_cholesky(raw11, raw21, raw22);
  const GfCov cov = gf_cov_from_chol(Lc);
  const GfRenderGeom rg = gf_render_geom(cov, p.normalize);
  const double S0 = acc8[0], S1 = acc8[1], S2 = acc8[2], S3 = acc8[3], S4 = acc8[4], S5 = acc8[5];
  const double a = (double)amp[g];
  const double nrm = (double)rg.norm;
  const double an = a * nrm;
  d_amp[g] = (float)(nrm * S0);
  d_mu[2 * g + 0] = (float)(an * (rg.i00 * S1 + rg.i01 * S2));
  d_mu[2 * g + 1] = (float)(an * (rg.i01 * S1 + rg.i11 * S2));
  const double G00 = -0.5 * an * S3, G01 = -0.5 * an * S4, G11 = -0.5 * an * S5;
  // AG = A G, AGA = A G A  (A, G symmetric)
  const double ag00 = rg.i00 * G00 + rg.i01 * G01, ag01 = rg.i00 * G01 + rg.i01 * G11;
  const double ag10 = rg.i01 * G00 + rg.i11 * G01, ag11 = rg.i01 * G01 + rg.i11 * G11;
  double c00 = -(ag00 * rg.i00 + ag01 * rg.i01);
  double c01 = -(ag00 * rg.i01 + ag01 * rg.i11);
  double c10 = -(ag10 * rg.i00 + ag11 * rg.i01);
  double c11 = -(ag10 * rg.i01 + ag11 * rg.i11);
  if (p.normalize) {
    const float sq = gf_sqrt_rn(rg.det_f);
    if (sq >= GF_FLT_EPS) {
      const double gdet = a * S0 * (-nrm / (2.0 * (double)rg.det_f));
      const double f = gdet * (double)rg.det_f;
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
  d_chol_raw[3 * g + 0] = (float)(dl11 * gf_softplus_grad(raw11));
  d_chol_raw[3 * g + 1] = (float)dl21;
  d_chol_raw[3 * g + 2] = (float)(dl22 * gf_softplus_grad(raw22));
}

template <typename TpIdx, typename GIdx>
__global__ __launch_bounds__(kTileThreads) void k_bwd_tiles(
    Problem p, const float* __restrict__ grad, const float* __restrict__ row_coords,
    const float* __restrict__ col_coords, const float* __restrict__ mu,
    const float* __restrict__ chol_raw, const float* __restrict__ amp,
    const TpIdx* __restrict__ tile_ptr, const GIdx* __restrict__ gids, int64_t num_pairs,
    float* __restrict__ d_mu, float* __restrict__ d_chol_raw, float* __restrict__ d_amp,
    uint8_t* ws, BwdLayout L) {
  __shared__ GaussLds gl[kTileThreads];
  __shared__ int32_t gid_lds[kTileThreads];
  __shared__ float red[kTileThreads / 64][8];
  __shared__ int is_last;
  WsHeader* hdr = reinterpret_cast<WsHeader*>(ws);
  float* acc = reinterpret_cast<float*>(ws + L.acc);
  const int64_t T = p.R * p.C;
  const int64_t t = blockIdx.x;
  const int lane = threadIdx.x & 63, wid = threadIdx.x >> 6;

  int64_t s = (int64_t)tile_ptr[t], e = (int64_t)tile_ptr[t + 1];
  if (threadIdx.x == 0) {
    if (s < 0 || e < s || e > num_pairs) set_status(&hdr->status, GF_STATUS_TILE_PTR_ORDER);
    if (t == T - 1 && e != num_pairs) set_status(&hdr->status, GF_STATUS_TILE_PTR_LAST);
  }
  if (s < 0) s = 0;
  if (e > num_pairs) e = num_pairs;
  const int64_t n = e > s ? e - s : 0;

  const int64_t tr = t / p.C, tc = t % p.C;
  const int64_t r0 = tr * p.tile_out, c0 = tc * p.tile_in;
  const int64_t r1 = (r0 + p.tile_out) < p.M ? (r0 + p.tile_out) : p.M;
  const int64_t c1 = (c0 + p.tile_in) < p.N ? (c0 + p.tile_in) : p.N;
  const int64_t w = c1 - c0;
  const int64_t npx = (r1 - r0) * w;

  for (int64_t j0 = 0; j0 < n; j0 += kTileThreads) {
    const int64_t nj = (n - j0) < kTileThreads ? (n - j0) : kTileThreads;
    __syncthreads();
    if (threadIdx.x < nj) {
      const int64_t g = (int64_t)gids[s + j0 + threadIdx.x];
      if (g < 0 || g >= p.K) {
        set_status(&hdr->status, g < 0 ? GF_STATUS_IDS_NEGATIVE : GF_STATUS_IDS_RANGE);
        gid_lds[threadIdx.x] = -1;
      } else {
        GeomF q;
        gaussian_geometry(p, mu, chol_raw, g, &q, nullptr);
        GaussLds v;
        v.mu0 = q.mu0;
        v.mu1 = q.mu1;
        v.i00 = q.i00;
        v.i01 = q.i01;
        v.i11 = q.i11;
        v.w = 0.0f;
        v.pad0 = v.pad1 = 0.0f;
        gl[threadIdx.x] = v;
        gid_lds[threadIdx.x] = (int32_t)g;
      }
    }
    __syncthreads();
    for (int j = 0; j < (int)nj; ++j) {
      const int32_t g = gid_lds[j];
      if (g < 0) continue;
      const GaussLds v = gl[j];
      float s0 = 0.f, s1 = 0.f, s2 = 0.f, s3 = 0.f, s4 = 0.f, s5 = 0.f;
      for (int64_t px = threadIdx.x; px < npx; px += kTileThreads) {
        const int64_t r = r0 + px / w, c = c0 + px % w;
        const float gr = grad[r * p.N + c];
        const float dx = row_coords[r] - v.mu0, dy = col_coords[c] - v.mu1;
        float q = (dx * v.i00 + dy * v.i01) * dx + (dx * v.i01 + dy * v.i11) * dy;
        bool live = true;
        if (p.has_clamp) {
          live = (q >= 0.0f) && (q <= p.clamp_quad);
          q = fminf(fmaxf(q, 0.0f), p.clamp_quad);
        }
        const float ge = gr * expf(-0.5f * q);
        s0 += ge;
        const float wv = live ? ge : 0.0f;
        s1 += wv * dx;
        s2 += wv * dy;
        s3 += wv * dx * dx;
        s4 += wv * dx * dy;
        s5 += wv * dy * dy;
      }
      s0 = wave_sum(s0);
      s1 = wave_sum(s1);
      s2 = wave_sum(s2);
      s3 = wave_sum(s3);
      s4 = wave_sum(s4);
      s5 = wave_sum(s5);
      if (lane == 0) {
        red[wid][0] = s0;
        red[wid][1] = s1;
        red[wid][2] = s2;
        red[wid][3] = s3;
        red[wid][4] = s4;
        red[wid][5] = s5;
      }
      __syncthreads();
      if (threadIdx.x < 6) {
        float tot = 0.f;
#pragma unroll
        for (int q = 0; q < kTileThreads / 64; ++q) tot += red[q][threadIdx.x];
        unsafeAtomicAdd(acc + 8 * (int64_t)g + threadIdx.x, tot);
      }
      __syncthreads();
    }
  }

  // Last workgroup applies the chain rule.
  __threadfence();
  __syncthreads();
  if (threadIdx.x == 0) {
    const uint32_t prev = atomicAdd(&hdr->ticket, 1u);
    is_last = (prev == (uint32_t)(gridDim.x - 1));
  }
  __syncthreads();
  if (!is_last) return;
  __threadfence();
  for (int64_t g = threadIdx.x; g < p.K; g += kTileThreads) {
    float a8[6];
#pragma unroll
    for (int q = 0; q < 6; ++q) {
      a8[q] = __hip_atomic_load(acc + 8 * g + q, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
      acc[8 * g + q] = 0.0f;  // leave the workspace zeroed for the next call
    }
    chain_one(p, mu, chol_raw, amp, a8, g, d_mu, d_chol_raw, d_amp);
  }
  if (threadIdx.x == 0) hdr->ticket = 0u;
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
  // wave reduction then one atomic per wave
#pragma unroll
  for (int o = 32; o > 0; o >>= 1) h += __shfl_xor(h, o, 64);
  if ((threadIdx.x & 63) == 0) atomicAdd(out, (unsigned long long)h);
}

// ------------------------------------------------------------------------------------------
// Host helpers.

int make_problem(const gf_field_config* cfg, int64_t M, int64_t N, int64_t K, Problem* p) {
  if (!cfg) return set_err(GF_E_INVALID_ARGUMENT, "config must not be NULL");
  if (cfg->tile_out <= 0) return set_err(GF_E_INVALID_ARGUMENT, "tile_out must be positive");
  if (cfg->tile_in <= 0) return set_err(GF_E_INVALID_ARGUMENT, "tile_in must be positive");
  if (!(cfg->sigma_multiplier > 0.0))
    return set_err(GF_E_INVALID_ARGUMENT, "sigma_multiplier must be positive");
  if (M <= 0 || N <= 0)
    return set_err(GF_E_INVALID_ARGUMENT, "out_features and in_features must be positive");
  if (K < 0) return set_err(GF_E_INVALID_ARGUMENT, "K must be non-negative");
  if (K > INT32_MAX) return set_err(GF_E_INVALID_ARGUMENT, "K must be < 2^31");
  p->M = M;
  p->N = N;
  p->K = K;
  p->tile_out = cfg->tile_out;
  p->tile_in = cfg->tile_in;
  p->R = (M + cfg->tile_out - 1) / cfg->tile_out;
  p->C = (N + cfg->tile_in - 1) / cfg->tile_in;
  if (p->R * p->C > INT32_MAX) return set_err(GF_E_INVALID_ARGUMENT, "too many tiles (>= 2^31)");
  p->sigma = (float)cfg->sigma_multiplier;
  p->clamp_quad = (float)cfg->clamp_quad;
  p->normalize = cfg->normalize ? 1 : 0;
  p->has_clamp = cfg->has_clamp_quad ? 1 : 0;
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
  return fwd_layout(k, p.R * p.C).total;
}

size_t gf_backward_workspace_bytes(int64_t out_features, int64_t in_features, int64_t k,
                                   const gf_field_config* cfg) {
  Problem p;
  if (make_problem(cfg, out_features, in_features, k, &p)) return 0;
  return bwd_layout(k).total;
}

int gf_forward_bin(const gf_field_config* cfg, int64_t out_features, int64_t in_features, int64_t k,
                   const float* mu, const float* chol_raw, int64_t* tile_ptr,
                   int64_t* num_pairs_dev, int64_t* num_pairs_host, void* workspace,
                   size_t workspace_bytes, void* stream) {
  Problem p;
  int rc = make_problem(cfg, out_features, in_features, k, &p);
  if (rc) return rc;
  const FwdLayout L = fwd_layout(k, p.R * p.C);
  if (!workspace || workspace_bytes < L.total)
    return set_err(GF_E_WORKSPACE, "forward workspace needs %zu bytes, got %zu", L.total, workspace_bytes);
  if (!tile_ptr || !num_pairs_dev) return set_err(GF_E_INVALID_ARGUMENT, "tile_ptr / num_pairs_dev must not be NULL");
  if (k > 0 && (!mu || !chol_raw)) return set_err(GF_E_INVALID_ARGUMENT, "mu / chol_raw must not be NULL");
  hipStream_t st = reinterpret_cast<hipStream_t>(stream);
  hipLaunchKernelGGL(k_bin, dim3(1), dim3(kBinThreads), 0, st, p, mu, chol_raw, tile_ptr,
                     num_pairs_dev, reinterpret_cast<uint8_t*>(workspace), L);
  GF_LAUNCH_CHECK("k_bin");
  if (num_pairs_host) {
    uint32_t status = 0;
    GF_HIP_CHECK(hipMemcpyAsync(num_pairs_host, num_pairs_dev, sizeof(int64_t), hipMemcpyDeviceToHost, st));
    GF_HIP_CHECK(hipMemcpyAsync(&status, workspace, sizeof(uint32_t), hipMemcpyDeviceToHost, st));
    GF_HIP_CHECK(hipStreamSynchronize(st));
    if (status & GF_STATUS_COUNT_MISMATCH)
      return set_err(GF_E_INTERNAL, "binning: per-tile counts disagree with per-Gaussian tile totals");
  }
  return GF_OK;
}

int gf_forward_render(const gf_field_config* cfg, int64_t out_features, int64_t in_features, int64_t k,
                      const float* row_coords, const float* col_coords, const float* mu,
                      const float* chol_raw, const float* amp, const int64_t* tile_ptr,
                      int64_t* gaussian_ids_sorted, int64_t ids_capacity, int64_t pairs_hint,
                      float* delta, void* workspace, size_t workspace_bytes, void* stream) {
  (void)mu;
  (void)chol_raw;
  Problem p;
  int rc = make_problem(cfg, out_features, in_features, k, &p);
  if (rc) return rc;
  const int64_t T = p.R * p.C;
  const FwdLayout L = fwd_layout(k, T);
  if (!workspace || workspace_bytes < L.total)
    return set_err(GF_E_WORKSPACE, "forward workspace needs %zu bytes, got %zu", L.total, workspace_bytes);
  if (!row_coords || !col_coords || !tile_ptr || !delta)
    return set_err(GF_E_INVALID_ARGUMENT, "coords / tile_ptr / delta must not be NULL");
  if (ids_capacity < 0 || (ids_capacity > 0 && !gaussian_ids_sorted))
    return set_err(GF_E_INVALID_ARGUMENT, "gaussian_ids_sorted / ids_capacity invalid");
  if (k > 0 && !amp) return set_err(GF_E_INVALID_ARGUMENT, "amp must not be NULL");
  hipStream_t st = reinterpret_cast<hipStream_t>(stream);
  uint8_t* ws = reinterpret_cast<uint8_t*>(workspace);
  if (k > 0) {
    int64_t work = pairs_hint > 0 ? pairs_hint : (ids_capacity > 0 ? ids_capacity : 1);
    int64_t blocks = (work + kEmitThreads - 1) / kEmitThreads;
    if (blocks < 1) blocks = 1;
    if (blocks > 65536) blocks = 65536;
    hipLaunchKernelGGL(k_emit, dim3((unsigned)blocks), dim3(kEmitThreads), 0, st, p, ws, L,
                       gaussian_ids_sorted, ids_capacity);
    GF_LAUNCH_CHECK("k_emit");
  }
  hipLaunchKernelGGL(k_render, dim3((unsigned)T), dim3(kTileThreads), 0, st, p, row_coords,
                     col_coords, amp, tile_ptr, gaussian_ids_sorted, ids_capacity, delta, ws, L);
  GF_LAUNCH_CHECK("k_render");
  return GF_OK;
}

int gf_backward(const gf_field_config* cfg, int64_t out_features, int64_t in_features, int64_t k,
                const float* grad_delta, const float* row_coords, const float* col_coords,
                const float* mu, const float* chol_raw, const float* amp, const void* tile_ptr,
                int32_t tile_ptr_is_int64, const void* gaussian_ids, int32_t ids_is_int64,
                int64_t num_pairs, float* d_mu, float* d_chol_raw, float* d_amp, void* workspace,
                size_t workspace_bytes, void* stream) {
  Problem p;
  int rc = make_problem(cfg, out_features, in_features, k, &p);
  if (rc) return rc;
  const int64_t T = p.R * p.C;
  const BwdLayout L = bwd_layout(k);
  if (!workspace || workspace_bytes < L.total)
    return set_err(GF_E_WORKSPACE, "backward workspace needs %zu bytes, got %zu", L.total, workspace_bytes);
  if (num_pairs < 0) return set_err(GF_E_INVALID_ARGUMENT, "num_pairs must be non-negative");
  if (!grad_delta || !row_coords || !col_coords || !tile_ptr)
    return set_err(GF_E_INVALID_ARGUMENT, "grad_delta / coords / tile_ptr must not be NULL");
  if (num_pairs > 0 && !gaussian_ids) return set_err(GF_E_INVALID_ARGUMENT, "gaussian_ids must not be NULL");
  if (k > 0 && (!mu || !chol_raw || !amp || !d_mu || !d_chol_raw || !d_amp))
    return set_err(GF_E_INVALID_ARGUMENT, "parameter / gradient pointers must not be NULL");
  hipStream_t st = reinterpret_cast<hipStream_t>(stream);
  uint8_t* ws = reinterpret_cast<uint8_t*>(workspace);
#define GF_BWD_LAUNCH(TP, GI)                                                                      \
  hipLaunchKernelGGL((k_bwd_tiles<TP, GI>), dim3((unsigned)T), dim3(kTileThreads), 0, st, p,      \
                     grad_delta, row_coords, col_coords, mu, chol_raw, amp,                       \
                     reinterpret_cast<const TP*>(tile_ptr), reinterpret_cast<const GI*>(gaussian_ids), \
                     num_pairs, d_mu, d_chol_raw, d_amp, ws, L)
  if (tile_ptr_is_int64 && ids_is_int64) GF_BWD_LAUNCH(int64_t, int64_t);
  else if (tile_ptr_is_int64) GF_BWD_LAUNCH(int64_t, int32_t);
  else if (ids_is_int64) GF_BWD_LAUNCH(int32_t, int64_t);
  else GF_BWD_LAUNCH(int32_t, int32_t);
#undef GF_BWD_LAUNCH
  GF_LAUNCH_CHECK("k_bwd_tiles");
  return GF_OK;
}

int gf_read_status(void* workspace, int32_t clear, uint32_t* status_host, void* stream) {
  if (!workspace || !status_host) return set_err(GF_E_INVALID_ARGUMENT, "workspace / status_host must not be NULL");
  hipStream_t st = reinterpret_cast<hipStream_t>(stream);
  WsHeader* hdr = reinterpret_cast<WsHeader*>(workspace);
  uint32_t v = 0;
  GF_HIP_CHECK(hipMemcpyAsync(&v, &hdr->status, sizeof(uint32_t), hipMemcpyDeviceToHost, st));
  GF_HIP_CHECK(hipStreamSynchronize(st));
  *status_host = v;
  if (clear) {
    GF_HIP_CHECK(hipMemsetAsync(&hdr->status, 0, sizeof(uint32_t), st));
  }
  return GF_OK;
}

int gf_selftest_softplus(uint64_t* checksum_host, void* stream) {
  if (!checksum_host) return set_err(GF_E_INVALID_ARGUMENT, "checksum_host must not be NULL");
  hipStream_t st = reinterpret_cast<hipStream_t>(stream);
  unsigned long long* d = nullptr;
  GF_HIP_CHECK(hipMalloc(&d, sizeof(unsigned long long)));
  hipError_t e = hipMemsetAsync(d, 0, sizeof(unsigned long long), st);
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
