/*
 * libm_sweep.c - test infrastructure (CPU only).
 *
 * Checks guass_amd/csrc/libm_f32.h (the restated expf / log1pf / softplus that the GPU
 * kernels use to bin Gaussians) against the host C library, which is what PyTorch's CPU
 * softplus calls on strided inputs (reference gaussian_peft/kernels/covariance.py:23,25).
 *
 *   libm_sweep [stride]      compare every stride-th float bit pattern (default 1 = all 2^32)
 *
 * Prints mismatch counts for expf (x in [-104, 20]), log1pf (y in [0, 4.9e8]) and the full
 * softplus over all inputs, plus an order-independent checksum of softplus(x) taken from the
 * host library: sum over x of mix64(bits(x) << 32 | bits(softplus(x))), NaN results
 * canonicalised.  The checksum over all 2^32 inputs is the golden value the GPU self-test
 * (gf_selftest_softplus) must reproduce.  Exit status 0 iff no mismatches.
 */
#include <math.h>
#include <stdint.h>
#include <stdio.h>
#include <stdlib.h>

#include "../guass_amd/csrc/libm_f32.h"

static uint64_t mix64(uint64_t z) {
  z += 0x9e3779b97f4a7c15ull;
  z = (z ^ (z >> 30)) * 0xbf58476d1ce4e5b9ull;
  z = (z ^ (z >> 27)) * 0x94d049bb133111ebull;
  return z ^ (z >> 31);
}

static uint32_t canon(float y) { return (y != y) ? 0x7fc00000u : gf_bits_f32(y); }

int main(int argc, char** argv) {
  const uint64_t stride = argc > 1 ? strtoull(argv[1], NULL, 10) : 1;
  uint64_t n_exp = 0, bad_exp = 0, n_log = 0, bad_log = 0, n_sp = 0, bad_sp = 0, hash = 0;
#pragma omp parallel for schedule(static) reduction(+ : n_exp, bad_exp, n_log, bad_log, n_sp, bad_sp, hash)
  for (int64_t i = 0; i < (int64_t)(0x100000000ull / stride); ++i) {
    const uint32_t u = (uint32_t)((uint64_t)i * stride);
    const float x = gf_f32_bits(u);
    if (x >= -104.0f && x <= 20.0f) {
      n_exp++;
      if (gf_bits_f32(expf(x)) != gf_bits_f32(gf_expf(x))) bad_exp++;
    }
    if (x >= 0.0f && x <= 4.9e8f) {
      n_log++;
      if (gf_bits_f32(log1pf(x)) != gf_bits_f32(gf_log1pf(x))) bad_log++;
    }
    const float ref = (x > 20.0f) ? x : log1pf(expf(x));
    const float mine = gf_softplus_torch_cpu(x);
    n_sp++;
    if (canon(ref) != canon(mine)) bad_sp++;
    hash += mix64(((uint64_t)u << 32) | canon(ref));
  }
  printf("stride=%llu expf: n=%llu mismatches=%llu\n", (unsigned long long)stride,
         (unsigned long long)n_exp, (unsigned long long)bad_exp);
  printf("log1pf: n=%llu mismatches=%llu\n", (unsigned long long)n_log, (unsigned long long)bad_log);
  printf("softplus: n=%llu mismatches=%llu\n", (unsigned long long)n_sp, (unsigned long long)bad_sp);
  printf("softplus_checksum=0x%016llx\n", (unsigned long long)hash);
  return (bad_exp || bad_log || bad_sp) ? 1 : 0;
}
