// fp32 exponential family used by every neuron/synapse kernel.
//
// The reference integrates with exp-Euler (brainstate/nn/_exp_euler.py:226-249):
//     x' = x + dt * exprel(dt * J) * f(x),    exprel(z) = (e^z - 1) / z
// and the Hodgkin-Huxley rates of examples/100_hh_neuron_model.py:49-64 call exp and
// exprel.  Device libm exp and glibc exp differ in the last ulp, and one ulp is enough
// to flip a threshold crossing, so spike rasters would not be reproducible against a
// CPU restatement.  These functions are built only from IEEE-754 +, -, *, /, fma and rint,
// all correctly rounded on gfx950 and on x86, so the same input gives the same bits on
// both sides (the library is compiled with -ffp-contract=off).
//
// Method (Cody & Waite, "Software Manual for the Elementary Functions", 1980):
//     n = rint(x * log2(e)),  r = fma(-n, L_lo, fma(-n, L_hi, x)),  |r| <= ln2/2
//     e^x = 2^n * P(r),  P = degree-7 Taylor polynomial of e^r (truncation < 6e-9),
//     evaluated by Horner's rule with fused multiply-adds
// L_hi = ln2 rounded to 16 significant bits (so n*L_hi is exact for |n| < 128) and
// L_lo = fl32(ln2 - L_hi).
#pragma once

#include <stdint.h>

#ifndef BS_HD
#define BS_HD __host__ __device__
#endif

#define BS_LOG2E_F ((float)1.4426950408889634)              /* fl32(1/ln 2) */
#define BS_LN2_HI_F 0.693145751953125f          /* 45426 / 2^16 */
#define BS_LN2_LO_F ((float)(0.6931471805599453 - 0.693145751953125)) /* fl32(ln 2 - L_hi) */
#define BS_EXP_XMAX 88.0f
#define BS_EXP_XMIN -87.0f
#define BS_EXPREL_SERIES 0.5f

BS_HD inline float bs_pow2i(int n) {
  // 2^n for n in [-126, 127] as a normal float, built from its bits.
  union { uint32_t u; float f; } v;
  v.u = (uint32_t)(n + 127) << 23;
  return v.f;
}

// a*b + c with one rounding (v_fma_f32 on the device, C99 fmaf on the host).  The library is
// built with -ffp-contract=off, so these are the only fused operations.
BS_HD inline float bs_fma(float a, float b, float c) { return __builtin_fmaf(a, b, c); }

BS_HD inline float bs_rint(float x) {
  // Round half to even (v_rndne_f32 on the device, nearbyintf on the host).
  return __builtin_rintf(x);
}

// e^x.  Inputs are clamped to [-87, 88]; below -87 the true value is < 1.7e-38 and
// the clamp returns ~1.65e-38 instead of a subnormal.
BS_HD inline float bs_expf(float x) {
  if (x > BS_EXP_XMAX) x = BS_EXP_XMAX;
  if (x < BS_EXP_XMIN) x = BS_EXP_XMIN;
  const float n = bs_rint(x * BS_LOG2E_F);
  float r = bs_fma(-n, BS_LN2_HI_F, x);
  r = bs_fma(-n, BS_LN2_LO_F, r);
  float p = (float)(1.0 / 5040.0);
  p = bs_fma(p, r, (float)(1.0 / 720.0));
  p = bs_fma(p, r, (float)(1.0 / 120.0));
  p = bs_fma(p, r, (float)(1.0 / 24.0));
  p = bs_fma(p, r, (float)(1.0 / 6.0));
  p = bs_fma(p, r, 0.5f);
  p = bs_fma(p, r, 1.0f);
  p = bs_fma(p, r, 1.0f);
  return p * bs_pow2i((int)n);
}

// exprel(z) = (e^z - 1) / z, with exprel(0) = 1.  For |z| < 1/2 the degree-7 Taylor
// series of exprel is used (truncation < 1.1e-8); elsewhere (e^z - 1) / z has no
// harmful cancellation.
// The series branch of bs_exprel (|z| < 1/2).
BS_HD inline float bs_exprel_series(float z) {
  float p = (float)(1.0 / 40320.0);
  p = bs_fma(p, z, (float)(1.0 / 5040.0));
  p = bs_fma(p, z, (float)(1.0 / 720.0));
  p = bs_fma(p, z, (float)(1.0 / 120.0));
  p = bs_fma(p, z, (float)(1.0 / 24.0));
  p = bs_fma(p, z, (float)(1.0 / 6.0));
  p = bs_fma(p, z, 0.5f);
  p = bs_fma(p, z, 1.0f);
  return p;
}

BS_HD inline float bs_exprel(float z) {
  float az = z < 0.0f ? -z : z;
  if (az < BS_EXPREL_SERIES) return bs_exprel_series(z);
  return (bs_expf(z) - 1.0f) / z;
}
