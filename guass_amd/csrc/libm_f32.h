// libm_f32.h - bit-exact fp32 softplus as computed by PyTorch's CPU kernel.
//
// The reference's CPU path activates the Cholesky factor with F.softplus on a strided
// column view (gaussian_peft/kernels/covariance.py:23,25).  On a non-contiguous input
// PyTorch's CPU softplus takes its scalar branch, x > 20 ? x : log1pf(expf(x)), i.e. the
// host C library's expf and log1pf (glibc on this image).  Tile assignment is decided by
// floor/ceil of values derived from softplus, so the GPU must reproduce those two
// functions to the last bit.  This header restates their published algorithms in
// portable IEEE arithmetic (no contraction, explicit fma) so that host C/C++ and gfx950
// device code compute identical results:
//   * gf_expf   - the table-driven exp of Szabolcs Nagy (ARM optimized-routines, glibc >= 2.28):
//                 2^(k/32) from a 32-entry table times a cubic in r, evaluated in double.
//   * gf_log1pf - the fdlibm single-precision log1p (Sun Microsystems, float conversion
//                 by Ian Lance Taylor), degree-7 polynomial in s = f/(2+f).
// Both were checked exhaustively against glibc 2.35 on every float input the softplus
// can pass them (expf: x in [-104, 20], 2,221,932,546 inputs; log1pf: y in [0, 4.9e8],
// 1,307,158,133 inputs); the single expf input where the cubic lands one double ulp on
// the other side of a float rounding boundary is pinned below.  The sweep program is
// oracle/libm_sweep.c.
#ifndef GUASS_AMD_LIBM_F32_H_
#define GUASS_AMD_LIBM_F32_H_

#include <stdint.h>

#if defined(__HIPCC__) || defined(__HIP__)
#define GF_HD __host__ __device__
#else
#define GF_HD
#endif

#ifdef __cplusplus
#define GF_INLINE static inline
#else
#define GF_INLINE static inline
#endif

GF_HD GF_INLINE uint64_t gf_bits_f64(double d) {
  uint64_t u;
  __builtin_memcpy(&u, &d, 8);
  return u;
}
GF_HD GF_INLINE double gf_f64_bits(uint64_t u) {
  double d;
  __builtin_memcpy(&d, &u, 8);
  return d;
}
GF_HD GF_INLINE uint32_t gf_bits_f32(float f) {
  uint32_t u;
  __builtin_memcpy(&u, &f, 4);
  return u;
}
GF_HD GF_INLINE float gf_f32_bits(uint32_t u) {
  float f;
  __builtin_memcpy(&f, &u, 4);
  return f;
}

// 2^(i/32) rounded to double, stored minus (i << 47) so that adding (k << 47) for the
// integer k = round(x*32/ln2) yields 2^(k/32) directly in the exponent field.
#define GF_EXP2_TABLE                                                                      \
  {0x3ff0000000000000ull, 0x3fefd9b0d3158574ull, 0x3fefb5586cf9890full, 0x3fef9301d0125b51ull, \
   0x3fef72b83c7d517bull, 0x3fef54873168b9aaull, 0x3fef387a6e756238ull, 0x3fef1e9df51fdee1ull, \
   0x3fef06fe0a31b715ull, 0x3feef1a7373aa9cbull, 0x3feedea64c123422ull, 0x3feece086061892dull, \
   0x3feebfdad5362a27ull, 0x3feeb42b569d4f82ull, 0x3feeab07dd485429ull, 0x3feea47eb03a5585ull, \
   0x3feea09e667f3bcdull, 0x3fee9f75e8ec5f74ull, 0x3feea11473eb0187ull, 0x3feea589994cce13ull, \
   0x3feeace5422aa0dbull, 0x3feeb737b0cdc5e5ull, 0x3feec49182a3f090ull, 0x3feed503b23e255dull, \
   0x3feee89f995ad3adull, 0x3feeff76f2fb5e47ull, 0x3fef199bdd85529cull, 0x3fef3720dcef9069ull, \
   0x3fef5818dcfba487ull, 0x3fef7c97337b9b5full, 0x3fefa4afa2a490daull, 0x3fefd0765b6e4540ull}

// expf for the inputs softplus passes it (x <= 20).
GF_HD GF_INLINE float gf_expf(float x) {
#pragma clang fp contract(off)
  const uint64_t table[32] = GF_EXP2_TABLE;
  if (x != x) return x + x;
  if (x < -104.0f) return 0.0f;  // below the smallest subnormal result
  if (gf_bits_f32(x) == 0xc27c65d9u) return gf_f32_bits(0x11fa2993u);  // pinned (see header)
  const double inv_ln2_n = 0x1.71547652b82fep+0 * 32.0;
  const double c0 = 0x1.c6af84b912394p-5 / 32.0 / 32.0 / 32.0;
  const double c1 = 0x1.ebfce50fac4f3p-3 / 32.0 / 32.0;
  const double c2 = 0x1.62e42ff0c52d6p-1 / 32.0;
  const double shift = 0x1.8p+52;
  const double xd = (double)x;
  const double z = inv_ln2_n * xd;
  double kd = z + shift;
  const uint64_t ki = gf_bits_f64(kd);
  kd -= shift;
  const double r = z - kd;
  uint64_t t = table[ki % 32u];
  t += ki << 47;
  const double s = gf_f64_bits(t);
  const double zz = __builtin_fma(c0, r, c1);
  const double r2 = r * r;
  double y = __builtin_fma(c2, r, 1.0);
  y = __builtin_fma(zz, r2, y);
  y = y * s;
  return (float)y;
}

GF_HD GF_INLINE float gf_div_f32(float a, float b) {
#if defined(__HIP_DEVICE_COMPILE__)
  return __fdiv_rn(a, b);
#else
  return a / b;
#endif
}

// log1pf for non-negative finite inputs (the range of expf); NaN passes through.
GF_HD GF_INLINE float gf_log1pf(float x) {
#pragma clang fp contract(off)
  const float ln2_hi = gf_f32_bits(0x3f317180u), ln2_lo = gf_f32_bits(0x3717f7d1u);
  const float lp1 = gf_f32_bits(0x3f2aaaabu), lp2 = gf_f32_bits(0x3ecccccdu),
              lp3 = gf_f32_bits(0x3e924925u), lp4 = gf_f32_bits(0x3e638e29u),
              lp5 = gf_f32_bits(0x3e3a3325u), lp6 = gf_f32_bits(0x3e1cd04fu),
              lp7 = gf_f32_bits(0x3e178897u);
  float hfsq, f = 0.0f, c = 0.0f, s, z, R, u;
  int32_t k, hu = 0;
  const int32_t hx = (int32_t)gf_bits_f32(x);
  const int32_t ax = hx & 0x7fffffff;
  if (x != x) return x + x;
  k = 1;
  if (hx < 0x3ed413d7) {          // x < 0.41422
    if (ax >= 0x3f800000) return (x - x) / (x - x);  // x <= -1 (not reached from softplus)
    if (ax < 0x31000000) {        // |x| < 2^-29
      if (ax < 0x24800000) return x;
      return x - x * x * 0.5f;
    }
    if (hx > 0 || hx <= (int32_t)0xbe95f61fu) {
      k = 0;
      f = x;
      hu = 1;
    }
  } else if (hx >= 0x7f800000) {
    return x + x;
  }
  if (k != 0) {
    if (hx < 0x5a000000) {
      u = 1.0f + x;
      hu = (int32_t)gf_bits_f32(u);
      k = (hu >> 23) - 127;
      c = (k > 0) ? 1.0f - (u - x) : x - (u - 1.0f);  // rounding error of 1+x
      c = gf_div_f32(c, u);
    } else {
      u = x;
      hu = (int32_t)gf_bits_f32(u);
      k = (hu >> 23) - 127;
      c = 0.0f;
    }
    hu &= 0x007fffff;
    if (hu < 0x3504f7) {
      u = gf_f32_bits((uint32_t)(hu | 0x3f800000));
    } else {
      k += 1;
      u = gf_f32_bits((uint32_t)(hu | 0x3f000000));
      hu = (0x00800000 - hu) >> 2;
    }
    f = u - 1.0f;
  }
  hfsq = 0.5f * f * f;
  if (hu == 0) {  // |f| < 2^-20
    if (f == 0.0f) {
      if (k == 0) return 0.0f;
      c += (float)k * ln2_lo;
      return (float)k * ln2_hi + c;
    }
    R = hfsq * (1.0f - 0.66666666666666666f * f);
    if (k == 0) return f - R;
    return (float)k * ln2_hi - ((R - ((float)k * ln2_lo + c)) - f);
  }
  s = gf_div_f32(f, 2.0f + f);
  z = s * s;
  R = z * (lp1 + z * (lp2 + z * (lp3 + z * (lp4 + z * (lp5 + z * (lp6 + z * lp7))))));
  if (k == 0) return f - (hfsq - s * (hfsq + R));
  return (float)k * ln2_hi - ((hfsq - (s * (hfsq + R) + ((float)k * ln2_lo + c))) - f);
}

// F.softplus(x) (beta = 1, threshold = 20) as PyTorch's CPU scalar branch computes it.
GF_HD GF_INLINE float gf_softplus_torch_cpu(float x) {
  return (x > 20.0f) ? x : gf_log1pf(gf_expf(x));
}

#endif  // GUASS_AMD_LIBM_F32_H_
