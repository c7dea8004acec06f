// host_geometry.cpp - host (x86-64, g++) build of the per-Gaussian geometry that the gfx950
// kernels run (geometry.h, libm_f32.h).  CPU tests compare it with the oracle to pin the
// binning arithmetic bit for bit without a GPU.  Not used by the product path.
#include <cstdint>

#include "geometry.h"

extern "C" {

// F.softplus as the reference CPU path computes it, elementwise.
void gfh_softplus(const float* x, float* y, int64_t n) {
  for (int64_t i = 0; i < n; ++i) y[i] = gf_softplus_torch_cpu(x[i]);
}

// Tile rectangles [K,4] = (r0, r1, c0, c1) and tiles touched [K] of K Gaussians.
void gfh_tile_rects(int64_t k, const float* mu, const float* chol_raw, int64_t M, int64_t N,
                    int64_t tile_out, int64_t tile_in, double sigma, int64_t* rects,
                    int64_t* touched) {
  const int64_t R = (M + tile_out - 1) / tile_out, C = (N + tile_in - 1) / tile_in;
  for (int64_t g = 0; g < k; ++g) {
    const GfChol L = gf_activate_cholesky(chol_raw[3 * g], chol_raw[3 * g + 1], chol_raw[3 * g + 2]);
    const GfCov c = gf_cov_from_chol(L);
    const GfRect r = gf_tile_rect(mu[2 * g], mu[2 * g + 1], c, M, N, tile_out, tile_in, R, C, (float)sigma);
    rects[4 * g + 0] = r.r0;
    rects[4 * g + 1] = r.r1;
    rects[4 * g + 2] = r.c0;
    rects[4 * g + 3] = r.c1;
    touched[g] = (r.r1 - r.r0 + 1) * (r.c1 - r.c0 + 1);
  }
}

// Activated Cholesky factor [K,3] = (l11, l21, l22) and fp32 covariance [K,3] = (s00, s01, s11).
void gfh_chol_cov(int64_t k, const float* chol_raw, float* chol, float* cov) {
  for (int64_t g = 0; g < k; ++g) {
    const GfChol L = gf_activate_cholesky(chol_raw[3 * g], chol_raw[3 * g + 1], chol_raw[3 * g + 2]);
    const GfCov c = gf_cov_from_chol(L);
    chol[3 * g + 0] = L.l11;
    chol[3 * g + 1] = L.l21;
    chol[3 * g + 2] = L.l22;
    cov[3 * g + 0] = c.s00;
    cov[3 * g + 1] = c.s01;
    cov[3 * g + 2] = c.s11;
  }
}

}  // extern "C"
