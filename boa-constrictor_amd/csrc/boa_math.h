// Device math shared by every kernel of the codec path.
//
// All code here is compiled with -ffp-contract=off: a multiply-add is fused
// only where __builtin_fmaf is written out.  The compress (chunk) and
// decompress (step) kernels call exactly these functions in the same order,
// which is what keeps their logits bit-identical (the decoder re-derives the
// encoder's integer CDFs from them).
//
// boa_expf / boa_logf are this project's own functions (not vendor libm):
//   exp: Cody-Waite reduction x = k ln2 + r with ln2 split in a float head and
//        tail, e^r by the degree-7 Taylor polynomial (Horner, fma), 2^k built
//        in the exponent field; x < -87 gives 0 so every result is normal.
//   log: y = 2^e m, m in [sqrt(1/2), sqrt(2)], log m = 2 atanh(s) with
//        s = (m-1)/(m+1), odd series to s^11.
// boa_repro_exp / tanh / gelu restate the reference's software activations
// (portability_solved_cpp/activations.hpp:33-117, device branch) operation
// for operation; the FF GELU of the reference uses them.
#pragma once
#include <hip/hip_runtime.h>
#include <stdint.h>

#define BOA_DEV __device__ __forceinline__

namespace boa {

BOA_DEV float u2f(uint32_t u) { return __uint_as_float(u); }
BOA_DEV uint32_t f2u(float f) { return __float_as_uint(f); }

BOA_DEV float expf_(float x) {
  if (x != x) return x;
  if (x > 88.72283935546875f) return __builtin_huge_valf();
  if (x < -87.0f) return 0.0f;
  const float LOG2E = 1.44269504088896340736f;
  const float LN2_HI = 0.693147182464599609375f;
  const float LN2_LO = -1.904654323148236e-09f;
  float kf = __builtin_rintf(x * LOG2E);
  float r = __builtin_fmaf(-kf, LN2_HI, x);
  r = __builtin_fmaf(-kf, LN2_LO, r);
  float p = 1.98412698412698412698e-4f;
  p = __builtin_fmaf(p, r, 1.38888888888888888889e-3f);
  p = __builtin_fmaf(p, r, 8.33333333333333333333e-3f);
  p = __builtin_fmaf(p, r, 4.16666666666666666667e-2f);
  p = __builtin_fmaf(p, r, 1.66666666666666666667e-1f);
  p = __builtin_fmaf(p, r, 0.5f);
  p = __builtin_fmaf(p, r, 1.0f);
  p = __builtin_fmaf(p, r, 1.0f);
  int k = (int)kf;
  if (k > 127) return (p * u2f((uint32_t)(127 + 127) << 23)) * 2.0f;
  return p * u2f((uint32_t)(k + 127) << 23);
}

BOA_DEV float logf_(float y) {
  if (y != y) return y;
  if (y == __builtin_huge_valf()) return y;
  if (y <= 0.0f) return (y == 0.0f) ? -__builtin_huge_valf() : __builtin_nanf("");
  uint32_t u = f2u(y);
  int e = (int)(u >> 23) - 127;
  if ((u >> 23) == 0) {
    y = y * 8388608.0f;
    u = f2u(y);
    e = (int)(u >> 23) - 127 - 23;
  }
  float m = u2f((u & 0x007FFFFFu) | 0x3F800000u);
  if (m > 1.41421353816986083984375f) { m = m * 0.5f; e += 1; }
  float s = (m - 1.0f) / (m + 1.0f);
  float s2 = s * s;
  float p = 0.0909090909090909090909f;
  p = __builtin_fmaf(p, s2, 0.111111111111111111111f);
  p = __builtin_fmaf(p, s2, 0.142857142857142857143f);
  p = __builtin_fmaf(p, s2, 0.2f);
  p = __builtin_fmaf(p, s2, 0.333333333333333333333f);
  float two_s = s + s;
  float lm = __builtin_fmaf(two_s * s2, p, two_s);
  const float LN2_HI = 0.693147182464599609375f;
  const float LN2_LO = -1.904654323148236e-09f;
  float ef = (float)e;
  return __builtin_fmaf(ef, LN2_HI, __builtin_fmaf(ef, LN2_LO, lm));
}

// activations.hpp:33-84 (device branch)
BOA_DEV float repro_exp(float x) {
  if (x <= -88.0f) return 0.0f;
  if (x >= 88.0f) x = 88.0f;
  float kf = __builtin_floorf(x * 1.44269504088896340736f + 0.5f);
  int k = (int)kf;
  float r = x + (-(kf * 0.69314718055994530942f));
  float t = 0.008333333333f + r * 0.001388888889f;
  t = 0.041666666667f + r * t;
  t = 0.166666666667f + r * t;
  t = 0.5f + r * t;
  t = 1.0f + r * t;
  t = 1.0f + r * t;
  return t * u2f((uint32_t)((k + 127) << 23));
}

// activations.hpp:87-98
BOA_DEV float repro_tanh(float x) {
  float ax = x < 0.0f ? -x : x;
  if (ax > 10.0f) return (x > 0.0f) ? 1.0f : -1.0f;
  float e2x = repro_exp(2.0f * x);
  return (e2x + -1.0f) / (e2x + 1.0f);
}

// activations.hpp:105-117 (tanh GELU used by the FF epilogue)
BOA_DEV float gelu(float x) {
  float cube = (x * x) * x;
  float inner = 0.79788456080286535588f * (x + 0.044715f * cube);
  float th = repro_tanh(inner);
  return 0.5f * (x * (1.0f + th));
}

// SiLU in the form v * (1 / (1 + exp(-v))) (mamba_kernels.cu:188-189)
BOA_DEV float silu(float x) {
  float sg = 1.0f / (1.0f + expf_(-x));
  return x * sg;
}

// unthresholded softplus log(1 + exp(x)) (inference_kernels.cu:376-382)
BOA_DEV float softplus(float x) { return logf_(1.0f + expf_(x)); }

}  // namespace boa
