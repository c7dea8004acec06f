// geometry.h - per-Gaussian geometry shared by the gfx950 kernels and their host build.
//
// Two kinds of result:
//  * the tile rectangle a Gaussian's sigma box covers.  It decides which (tile, gaussian)
//    pairs exist and must equal the reference CPU path bit for bit, so it follows that
//    path's fp32 operation sequence exactly (no contraction, correctly rounded sqrt):
//      covariance.py:14-26  L = [[softplus(r11)+eps, 0], [r21, softplus(r22)+eps]]
//      bounds.py:44-58      cov = L L^T (small-matrix bmm: each entry ((0 + a0*b0) + a1*b1)),
//                           std = sqrt(max(cov_ii, 1e-8)), centre = (mu+1)*0.5*(M-1),
//                           half = sigma*std*0.5*max(M-1,1), floor/ceil, clamp, / tile.
//  * the render geometry (inverse covariance, determinant, normalisation).  The reference
//    CPU path takes torch.linalg.inv / det of the same fp32 cov (gaussian_core.py:42-44);
//    here the 2x2 inverse of that fp32 matrix is formed in double and rounded once.  The
//    reference CUDA kernel instead clamps det at 1e-8 before inverting (forward.cu:171-176),
//    which changes the field of every Gaussian with det(cov) < 1e-8; the CPU path, which is
//    the parity target, has no such clamp and neither does this code.
#ifndef GUASS_AMD_GEOMETRY_H_
#define GUASS_AMD_GEOMETRY_H_

#include <stdint.h>

#include "libm_f32.h"

#define GF_CHOL_EPS 1e-5f
#define GF_COV_FLOOR 1e-8f
#define GF_FLT_EPS 1.1920928955078125e-07f /* torch.finfo(float32).eps */
#define GF_TWO_PI_F32 6.2831854820251465f  /* float(2*pi) as a scalar multiplies fp32 */

typedef struct GfChol {
  float l11, l21, l22;
} GfChol;

typedef struct GfCov {
  float s00, s01, s11;  // fp32 cov = L L^T entries (s10 == s01)
} GfCov;

typedef struct GfRect {
  int64_t r0, r1, c0, c1;  // inclusive tile ranges
} GfRect;

// One diagonal entry of the Cholesky factor: softplus(raw) + eps, the sum rounded on its own.
GF_HD GF_INLINE float gf_activate_diag(float raw) {
#pragma clang fp contract(off)
  return gf_softplus_torch_cpu(raw) + GF_CHOL_EPS;
}

GF_HD GF_INLINE GfChol gf_activate_cholesky(float raw11, float raw21, float raw22) {
  GfChol L;
  L.l11 = gf_activate_diag(raw11);
  L.l21 = raw21;
  L.l22 = gf_activate_diag(raw22);
  return L;
}

GF_HD GF_INLINE GfCov gf_cov_from_chol(GfChol L) {
#pragma clang fp contract(off)
  GfCov c;
  // (L L^T)_ij = (0 + L_i0 * L_j0) + L_i1 * L_j1 with L_01 = 0.
  c.s00 = (0.0f + L.l11 * L.l11) + 0.0f * 0.0f;
  c.s01 = (0.0f + L.l11 * L.l21) + 0.0f * L.l22;
  c.s11 = (0.0f + L.l21 * L.l21) + L.l22 * L.l22;
  return c;
}

// PyTorch's CPU float -> int64 cast (cvttss2si): NaN and out-of-range give INT64_MIN.
GF_HD GF_INLINE int64_t gf_f32_to_i64_torch(float x) {
  if (!(x >= -0x1p63f && x < 0x1p63f)) return INT64_MIN;
  return (int64_t)x;
}

GF_HD GF_INLINE int64_t gf_clamp_i64(int64_t v, int64_t lo, int64_t hi) {
  return v < lo ? lo : (v > hi ? hi : v);
}

// IEEE sqrt, correctly rounded, on host and device alike.  On the device this is the LLVM sqrt,
// which HIP lowers to the correctly rounded sequence (v_sqrt_f32 and a one-ulp correction);
// HIP's __fsqrt_rn is the native v_sqrt_f32 unless OCML_BASIC_ROUNDED_OPERATIONS is defined,
// which is off by one ulp for some inputs.
GF_HD GF_INLINE float gf_sqrt_rn(float x) { return __builtin_sqrtf(x); }

// torch.clamp(x, min=lo) keeps NaN.
GF_HD GF_INLINE float gf_clamp_min_nan(float x, float lo) { return (x != x) ? x : (x < lo ? lo : x); }

GF_HD GF_INLINE GfRect gf_tile_rect(float mu0, float mu1, GfCov c, int64_t M, int64_t N,
                                    int64_t tile_out, int64_t tile_in, int64_t R, int64_t C,
                                    float sigma) {
#pragma clang fp contract(off)
  const float std_r = gf_sqrt_rn(gf_clamp_min_nan(c.s00, GF_COV_FLOOR));
  const float std_c = gf_sqrt_rn(gf_clamp_min_nan(c.s11, GF_COV_FLOOR));
  const float centre_r = ((mu0 + 1.0f) * 0.5f) * (float)(M - 1);
  const float centre_c = ((mu1 + 1.0f) * 0.5f) * (float)(N - 1);
  const float half_r = ((sigma * std_r) * 0.5f) * (float)(M - 1 > 1 ? M - 1 : 1);
  const float half_c = ((sigma * std_c) * 0.5f) * (float)(N - 1 > 1 ? N - 1 : 1);
  const int64_t row_lo = gf_clamp_i64(gf_f32_to_i64_torch(__builtin_floorf(centre_r - half_r)), 0, M - 1);
  const int64_t row_hi = gf_clamp_i64(gf_f32_to_i64_torch(__builtin_ceilf(centre_r + half_r)), 0, M - 1);
  const int64_t col_lo = gf_clamp_i64(gf_f32_to_i64_torch(__builtin_floorf(centre_c - half_c)), 0, N - 1);
  const int64_t col_hi = gf_clamp_i64(gf_f32_to_i64_torch(__builtin_ceilf(centre_c + half_c)), 0, N - 1);
  GfRect r;
  r.r0 = gf_clamp_i64(row_lo / tile_out, 0, R - 1);
  r.r1 = gf_clamp_i64(row_hi / tile_out, 0, R - 1);
  r.c0 = gf_clamp_i64(col_lo / tile_in, 0, C - 1);
  r.c1 = gf_clamp_i64(col_hi / tile_in, 0, C - 1);
  return r;
}

typedef struct GfRenderGeom {
  double i00, i01, i11;  // inverse of the fp32 cov
  double det;            // det of the fp32 cov
  float norm;            // 1/(2*pi*max(sqrt(det), eps)) if normalize, else 1
  float det_f;           // det rounded to fp32
} GfRenderGeom;

GF_HD GF_INLINE GfRenderGeom gf_render_geom(GfCov c, int normalize) {
  GfRenderGeom g;
  const double a = (double)c.s00, b = (double)c.s01, d = (double)c.s11;
  const double det = a * d - b * b;  // the two products are exact in double
  g.det = det;
  g.i00 = d / det;
  g.i01 = -b / det;
  g.i11 = a / det;
  g.det_f = (float)det;
  if (normalize) {
#pragma clang fp contract(off)
    const float s = gf_sqrt_rn(g.det_f);
    const float sc = (s < GF_FLT_EPS) ? GF_FLT_EPS : s;
    g.norm = gf_div_f32(1.0f, GF_TWO_PI_F32 * sc);
  } else {
    g.norm = 1.0f;
  }
  return g;
}

GF_HD GF_INLINE double gf_exp_f64(double x) {
#if defined(__HIP_DEVICE_COMPILE__)
  return exp(x);
#else
  return __builtin_exp(x);
#endif
}

// d softplus / dx as PyTorch's softplus backward computes it: x > 20 ? 1 : e^x / (e^x + 1).
GF_HD GF_INLINE double gf_softplus_grad(float x) {
  if (x > 20.0f) return 1.0;
  const double z = gf_exp_f64((double)x);
  return z / (z + 1.0);
}

#endif  // GUASS_AMD_GEOMETRY_H_
