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

// bfloat16 storage (uint16_t): the upper half of a float32, rounded to
// nearest even by gfx950's v_cvt_pk_bf16_f32; a NaN stays a quiet NaN.
BOA_DEV uint16_t f32_to_bf16(float x) { return __builtin_bit_cast(uint16_t, (__bf16)x); }
BOA_DEV float bf16_to_f32(uint16_t h) { return u2f((uint32_t)h << 16); }
BOA_DEV float bf16r(float x) { return bf16_to_f32(f32_to_bf16(x)); }

// activation storage: fp32 or bf16
BOA_DEV float ldv(const float* p) { return *p; }
BOA_DEV float ldv(const uint16_t* p) { return bf16_to_f32(*p); }
BOA_DEV void stv(float* p, float v) { *p = v; }
BOA_DEV void stv(uint16_t* p, float v) { *p = f32_to_bf16(v); }

// e^x and log(y) in two forms with identical results for every input:
// expf_ / logf_ are branch-free (the arithmetic runs on a clamped or rescaled
// argument and selects give the special values, so a wavefront never
// diverges), expf_br / logf_br return early on special values.  2^k is
// applied with ldexp, which is exact here as the product with 2^k is (for
// k = 128 either form overflows alike).  Long per-element chains (the chunk
// scan) run faster branch-free; latency-bound kernels (the decode step) run
// faster with the early returns.

// e^x for finite x in [-87, 88.7228...]
BOA_DEV float exp_core(float x) {
  const float LOG2E = 1.44269504088896340736f;
  const float LN2_HI = 0.693147182464599609375f;
  const float LN2_LO = -1.904654323148236e-09f;
  const float kf = __builtin_rintf(x * LOG2E);
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
  return __builtin_ldexpf(p, (int)kf);
}

BOA_DEV float expf_(float x) {
  float res = exp_core(__builtin_fminf(__builtin_fmaxf(x, -87.0f), 88.72283935546875f));
  res = x < -87.0f ? 0.0f : res;
  res = x > 88.72283935546875f ? __builtin_huge_valf() : res;
  return x != x ? x : res;
}

// 2^t for t <= 0, the exponentials whose argument is never positive: the
// selective scan's decay exp(-exp(A_log) dt), taken in base 2 (the weights
// hold na2 = -exp(A_log) * log2(e), two fp32 roundings done once at load,
// and the scan takes 2^t of t = na2 * dt), and the CDF's exp(l - max),
// taken as 2^((l - max) log2(e)).  t is clamped into
// [-126, 0] (fmaxf turns a NaN into -126), split as k + r with k = rint(t)
// and r = t - k in [-1/2, 1/2] (exact); 2^r comes from a degree-6
// polynomial with 2^0 = 1 exact, fitted to the relative error of 2^r on
// [-1/2, 1/2] (under one ulp with fp32 fma evaluation), and 2^k is applied
// with ldexp.  The least result is 2^-126: no subnormal is produced.
BOA_DEV float exp2_neg(float t) {
  const float s = __builtin_fminf(__builtin_fmaxf(t, -126.0f), 0.0f);
  const float k = __builtin_rintf(s);
  const float r = s - k;
  float p = 0x1.41fbbap-13f;
  p = __builtin_fmaf(p, r, 0x1.5f3e54p-10f);
  p = __builtin_fmaf(p, r, 0x1.3b2d4cp-7f);
  p = __builtin_fmaf(p, r, 0x1.c6aee8p-5f);
  p = __builtin_fmaf(p, r, 0x1.ebfbdcp-3f);
  p = __builtin_fmaf(p, r, 0x1.62e430p-1f);
  p = __builtin_fmaf(p, r, 1.0f);
  return __builtin_ldexpf(p, (int)k);
}

BOA_DEV float expf_br(float x) {
  if (x != x) return x;
  if (x > 88.72283935546875f) return __builtin_huge_valf();
  if (x < -87.0f) return 0.0f;
  return exp_core(x);
}

// log(y) for y > 0 finite (subnormals rescaled)
BOA_DEV float log_core(float y) {
  const bool sub = (f2u(y) >> 23) == 0;
  const uint32_t u = f2u(sub ? y * 8388608.0f : y);
  int e = (int)(u >> 23) - 127 - (sub ? 23 : 0);
  float m = u2f((u & 0x007FFFFFu) | 0x3F800000u);
  const bool hi = m > 1.41421353816986083984375f;
  m = hi ? m * 0.5f : m;
  e = hi ? e + 1 : e;
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

BOA_DEV float logf_(float y) {
  float res = log_core(y);
  res = y == 0.0f ? -__builtin_huge_valf() : res;
  res = y < 0.0f ? __builtin_nanf("") : res;
  res = y == __builtin_huge_valf() ? y : res;
  return y != y ? y : res;
}

BOA_DEV float logf_br(float y) {
  if (y != y) return y;
  if (y == __builtin_huge_valf()) return y;
  if (y <= 0.0f) return (y == 0.0f) ? -__builtin_huge_valf() : __builtin_nanf("");
  return log_core(y);
}

// Forms of the transcendental activations.  MATH_BF and MATH_BR give
// identical results (branch-free vs early-return special cases; the
// oracle's functions).  MATH_HW uses the hardware exp2/log2/reciprocal
// (v_exp_f32, v_log_f32, v_rcp_f32, about 1 ulp): the bf16 precision runs on
// it in compress and decode alike, so its two passes still agree bit for
// bit while its logits are compared with the oracle within the bf16
// tolerance.
enum { MATH_BF = 0, MATH_BR = 1, MATH_HW = 2 };

BOA_DEV float hw_exp(float x) { return __builtin_amdgcn_exp2f(x * 1.44269504088896340736f); }
BOA_DEV float hw_log(float x) { return __builtin_amdgcn_logf(x) * 0.69314718055994530942f; }
BOA_DEV float hw_rcp(float x) { return __builtin_amdgcn_rcpf(x); }

template <int M>
BOA_DEV float exp_sel(float x) { return M == MATH_HW ? hw_exp(x) : M == MATH_BR ? expf_br(x) : expf_(x); }
template <int M>
BOA_DEV float log_sel(float x) { return M == MATH_HW ? hw_log(x) : M == MATH_BR ? logf_br(x) : logf_(x); }
template <int M>
BOA_DEV float rcp_sel(float x) { return M == MATH_HW ? hw_rcp(x) : 1.0f / x; }

// activations.hpp:33-84 (device branch); core for x in [-88, 88]
BOA_DEV float repro_exp_core(float x) {
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

template <int M>
BOA_DEV float repro_exp(float x) {
  if (M == MATH_HW) return hw_exp(x);
  if (M == MATH_BR) {
    if (x <= -88.0f) return 0.0f;
    return repro_exp_core(x >= 88.0f ? 88.0f : x);
  }
  const float res = repro_exp_core(__builtin_fminf(__builtin_fmaxf(x, -88.0f), 88.0f));
  return x <= -88.0f ? 0.0f : (x != x ? x : res);
}

// activations.hpp:87-98
template <int M>
BOA_DEV float repro_tanh(float x) {
  const float ax = x < 0.0f ? -x : x;
  if (M == MATH_BR && ax > 10.0f) return (x > 0.0f) ? 1.0f : -1.0f;
  const float e2x = repro_exp<M>(2.0f * x);
  const float th = M == MATH_HW ? 1.0f - 2.0f * hw_rcp(e2x + 1.0f) : (e2x + -1.0f) / (e2x + 1.0f);
  return ax > 10.0f ? ((x > 0.0f) ? 1.0f : -1.0f) : th;
}

// activations.hpp:105-117 (tanh GELU used by the FF epilogue)
template <int M = MATH_BF>
BOA_DEV float gelu(float x) {
  float cube = (x * x) * x;
  float inner = 0.79788456080286535588f * (x + 0.044715f * cube);
  float th = repro_tanh<M>(inner);
  return 0.5f * (x * (1.0f + th));
}

// SiLU in the form v * (1 / (1 + exp(-v))) (mamba_kernels.cu:188-189)
template <int M = MATH_BF>
BOA_DEV float silu(float x) {
  float sg = rcp_sel<M>(1.0f + exp_sel<M>(-x));
  return x * sg;
}

// unthresholded softplus log(1 + exp(x)) (inference_kernels.cu:376-382)
template <int M = MATH_BF>
BOA_DEV float softplus(float x) { return log_sel<M>(1.0f + exp_sel<M>(x)); }

// 2^t for t <= 0 (see exp2_neg) in the chosen form
template <int M>
BOA_DEV float exp2_neg_sel(float t) {
  return M == MATH_HW ? __builtin_amdgcn_exp2f(t) : exp2_neg(t);
}

// the scan's base-2 decay coefficient from A_log (see exp2_neg)
BOA_DEV float scan_na2(float a_log) { return -expf_(a_log) * 1.44269504088896340736f; }

}  // namespace boa
