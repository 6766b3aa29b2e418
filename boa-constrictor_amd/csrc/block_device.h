// Per-element device code shared by the chunk (compress) and step (decode)
// kernels: the causal conv value and the fused dt_proj + softplus + scan +
// D + gate of one token of one channel.  Both paths call these functions,
// which is what keeps their results bit-identical.
#pragma once
#include "boa_kernels.h"

namespace boa {

// value = bias + x[t-3] w0 + x[t-2] w1 + x[t-1] w2 + x[t] w3 (unfused, k
// order), then SiLU.  The state holds the last four inputs, most recent last.
template <int M = MATH_BF>
__device__ __forceinline__ float conv_value(float bias, float xm3, float xm2, float xm1, float x0,
                                            const float4 w) {
  float v = bias;
  v = v + xm3 * w.x;
  v = v + xm2 * w.y;
  v = v + xm1 * w.z;
  v = v + x0 * w.w;
  return silu<M>(v);
}

// Step form: state s = (x[t-4], x[t-3], x[t-2], x[t-1]), new input x0.
template <int M = MATH_BF>
__device__ __forceinline__ float conv_step_value(float bias, float4 s, float x0, const float4 w) {
  return conv_value<M>(bias, s.y, s.z, s.w, x0, w);
}

// Decode-step activation layouts, lane capacity ld:
//   fp32 "k-blocked": feature k of lane m at ((k/16) ld + m) 16 + dperm(k%16),
//     dperm(j) = 4 (j%4) + j/4 (a 4x4 transpose, its own inverse), so that the
//     four k-steps of a 16x16x4 MFMA operand are one float4 of the lane;
//   bf16 "32-blocked": feature k of lane m at ((k/32) ld + m) 32 + k%32, so
//     that the 8 k of a 16x16x32 bf16 MFMA operand slot group are 16 bytes.
__device__ __forceinline__ int dperm(int j) { return ((j & 3) << 2) | ((j >> 2) & 3); }

// Streaming (nontemporal) access to the decode step's recurrent state, which
// every step reads and rewrites once per layer (more than the last-level
// cache holds), so that it does not evict the weights and activations.
typedef float stream_f4 __attribute__((ext_vector_type(4)));
__device__ __forceinline__ float4 ld_stream(const float4* p) {
  const stream_f4 v = __builtin_nontemporal_load(reinterpret_cast<const stream_f4*>(p));
  return make_float4(v[0], v[1], v[2], v[3]);
}
__device__ __forceinline__ void st_stream(float4* p, float4 v) {
  __builtin_nontemporal_store(stream_f4{v.x, v.y, v.z, v.w}, reinterpret_cast<stream_f4*>(p));
}
// State of the layers that fit in the last-level cache next to the weights
// uses ordinary (cached) accesses; the rest is streamed.
__device__ __forceinline__ float4 state_ld4(const float4* p, bool cached) {
  return cached ? *p : ld_stream(p);
}
__device__ __forceinline__ void state_st4(float4* p, float4 v, bool cached) {
  if (cached) *p = v;
  else st_stream(p, v);
}
// The conv step reads the last three of a channel's four state values (the
// oldest drops out): loading only those keeps the compiler from reusing the
// fourth one's register while its load is in flight, which it guards with a
// wait for that load and every load before it.  x is left 0.
typedef float stream_f3 __attribute__((ext_vector_type(3)));
template <bool CACHED>
__device__ __forceinline__ float4 state_ld3(const float4* p) {
  const stream_f3* q = reinterpret_cast<const stream_f3*>(reinterpret_cast<const float*>(p) + 1);
  const stream_f3 v = CACHED ? *q : __builtin_nontemporal_load(q);
  return make_float4(0.0f, v[0], v[1], v[2]);
}
// bf16 precision keeps the step-layout conv state as four bf16 (8 bytes) per
// channel and lane: its values are the bf16-rounded in_proj outputs, so the
// narrow form is exact and halves the state's traffic.
typedef unsigned short stream_h4 __attribute__((ext_vector_type(4)));
__device__ __forceinline__ float4 state_ld4h(const ushort4* p, bool cached) {
  stream_h4 v;
  if (cached) {
    const ushort4 t = *p;
    v = stream_h4{t.x, t.y, t.z, t.w};
  } else {
    v = __builtin_nontemporal_load(reinterpret_cast<const stream_h4*>(p));
  }
  return make_float4(bf16_to_f32(v[0]), bf16_to_f32(v[1]), bf16_to_f32(v[2]), bf16_to_f32(v[3]));
}
__device__ __forceinline__ void state_st4h(ushort4* p, float4 f, bool cached) {
  const stream_h4 v{f32_to_bf16(f.x), f32_to_bf16(f.y), f32_to_bf16(f.z), f32_to_bf16(f.w)};
  if (cached) *p = make_ushort4(v[0], v[1], v[2], v[3]);
  else __builtin_nontemporal_store(v, reinterpret_cast<stream_h4*>(p));
}
__device__ __forceinline__ size_t dblk(int k, int m, int ld) {
  return ((size_t)(k >> 4) * ld + m) * 16 + dperm(k & 15);
}
__device__ __forceinline__ size_t dblk32(int k, int m, int ld) {
  return ((size_t)(k >> 5) * ld + m) * 32 + (k & 31);
}

// Staged-operand pipelines fed by direct-to-LDS copies (global_load_lds):
// the compiler counts such a copy as an LDS write and waits for every copy
// in flight (vmcnt(0)) before any LDS read it emits, and __syncthreads()
// waits for them too; both would drain the pipeline every stage.  These
// reads and this barrier are outside its view: the caller waits for the
// copies it needs (s_waitcnt vmcnt(n)) before lds_barrier, and for its reads
// with lds_wait4 before using them.
typedef uint32_t lds_u32x4 __attribute__((ext_vector_type(4)));
__device__ __forceinline__ lds_u32x4 lds_read128(const void* p) {
  lds_u32x4 v;
  const uint32_t a = (uint32_t)(uintptr_t)(const __attribute__((address_space(3))) void*)p;
  asm volatile("ds_read_b128 %0, %1" : "=v"(v) : "v"(a) : "memory");
  return v;
}
__device__ __forceinline__ void lds_barrier() { asm volatile("s_barrier" ::: "memory"); }
// the reads' values are the asm's outputs, so nothing uses them before it
__device__ __forceinline__ void lds_wait4(lds_u32x4& a, lds_u32x4& b, lds_u32x4& c, lds_u32x4& d) {
  asm volatile("s_waitcnt lgkmcnt(0)" : "+v"(a), "+v"(b), "+v"(c), "+v"(d)::"memory");
}
__device__ __forceinline__ void lds_wait8(lds_u32x4& a, lds_u32x4& b, lds_u32x4& c, lds_u32x4& d,
                                          lds_u32x4& e, lds_u32x4& f, lds_u32x4& g, lds_u32x4& h) {
  asm volatile("s_waitcnt lgkmcnt(0)"
               : "+v"(a), "+v"(b), "+v"(c), "+v"(d), "+v"(e), "+v"(f), "+v"(g), "+v"(h)::"memory");
}
// s_waitcnt vmcnt(n) for the n a staged loop allows (its immediates)
__device__ __forceinline__ void vm_wait(int n) {
  switch (n) {
    case 24: asm volatile("s_waitcnt vmcnt(24)" ::: "memory"); break;
    case 20: asm volatile("s_waitcnt vmcnt(20)" ::: "memory"); break;
    case 16: asm volatile("s_waitcnt vmcnt(16)" ::: "memory"); break;
    case 10: asm volatile("s_waitcnt vmcnt(10)" ::: "memory"); break;
    case 8: asm volatile("s_waitcnt vmcnt(8)" ::: "memory"); break;
    case 5: asm volatile("s_waitcnt vmcnt(5)" ::: "memory"); break;
    case 4: asm volatile("s_waitcnt vmcnt(4)" ::: "memory"); break;
    case 2: asm volatile("s_waitcnt vmcnt(2)" ::: "memory"); break;
    default: asm volatile("s_waitcnt vmcnt(0)" ::: "memory"); break;
  }
}

// (lane block, feature block) of 128 x 128 GEMM block b.  Workgroups go to
// the eight XCDs round-robin (b % 8); when the lane blocks divide by eight,
// XCD x takes lane blocks x, x + 8, ... with every feature block, so that
// each XCD's L2 holds an eighth of the activations and in_proj's conv
// blocks (the first feature blocks) spread over every XCD instead of
// landing on XCDs 0-3.
__device__ __forceinline__ int2 t128_block(int b, int m_blocks, int n_blocks) {
  if (m_blocks % 8) return make_int2(b / n_blocks, b % n_blocks);
  const int x = b & 7, k = b >> 3;
  return make_int2(8 * (k / n_blocks) + x, k % n_blocks);
}

constexpr int RMAX = 32;  // dt_rank <= 32 (d_model <= 512)

template <int DS, int RB>
struct ScanCtx {
  float wdt[RB];
  float na[DS];
  float h[DS];
  float bdt, dd;
};

template <int DS, int RB>
__device__ __forceinline__ void scan_load(ScanCtx<DS, RB>& sc, const LayerW& Lw, const float* ssm,
                                          int c, int di, int r) {
#pragma unroll
  for (int j = 0; j < RB; ++j) sc.wdt[j] = j < r ? Lw.w_dt[(size_t)j * di + c] : 0.0f;
#pragma unroll
  for (int n = 0; n < DS; n += 4) {
    float4 a = *reinterpret_cast<const float4*>(Lw.na2 + (size_t)c * DS + n);
    sc.na[n] = a.x; sc.na[n + 1] = a.y; sc.na[n + 2] = a.z; sc.na[n + 3] = a.w;
    float4 hv = *reinterpret_cast<const float4*>(ssm + n);
    sc.h[n] = hv.x; sc.h[n + 1] = hv.y; sc.h[n + 2] = hv.z; sc.h[n + 3] = hv.w;
  }
  sc.bdt = Lw.b_dt[c];
  sc.dd = Lw.dd[c];
}

template <int DS, int RB>
__device__ __forceinline__ void scan_store(const ScanCtx<DS, RB>& sc, float* ssm) {
#pragma unroll
  for (int n = 0; n < DS; n += 4)
    *reinterpret_cast<float4*>(ssm + n) = make_float4(sc.h[n], sc.h[n + 1], sc.h[n + 2], sc.h[n + 3]);
}

// One token of one channel: dt = softplus(delta[0:r] . w_dt[:, c] + b_dt),
// h_n = exp(-exp(A_log) dt) h_n + (dt B_n) u, y = sum_n h_n C_n + D u,
// (the decay taken as 2^(na2_n dt), na2 = -exp(A_log) log2(e)),
// out = y * (z * sigmoid(z)).  M selects the exp/log form (MATH_BF and
// MATH_BR give the same results).
// The update rounds every product and sum on its own, as the reference's
// __fmul_rn / __fadd_rn lines do (mamba_kernels.cu:332-335, 453-461):
// dB = dt B_n, h_n = (dA h_n) + (dB u), y = y + (h_n C_n); the build's
// -ffp-contract=off keeps the compiler from fusing them.  The bf16 precision
// (M = MATH_HW, hardware transcendentals, results within the bf16
// tolerance of the oracle rather than bit-equal) takes the fused form
// h_n = fma(dA, h_n, B_n (dt u)), y = fma(h_n, C_n, y): three VALU
// operations fewer per state; compress and decode both run this function,
// so their bits still agree.
// The fused form at d_state 16 only: at d_state 32 its compress scan needs
// 140 VGPRs (three waves per SIMD) against 127 unfused (four), and measured
// slower on the C5 probe (compress scan 937 against 836 ms; capped at four
// waves it spills, 1126 ms), while its decode scan was 4 % faster.
#ifndef BOA_SCAN_B16_FUSED_DS32
#define BOA_SCAN_B16_FUSED_DS32 0
#endif
template <int DS, int M>
constexpr bool scan_fused_update() {
  return M == MATH_HW && (DS == 16 || BOA_SCAN_B16_FUSED_DS32);
}
// The channel's parameters come from P: wdt(j), na(n), bdt(), dd() (the
// registers of a ScanCtx, or shared memory); h is updated in place.
template <int DS, int RB, int M, class P>
__device__ __forceinline__ float scan_token_p(float (&h)[DS], const P& p, const float* dt_in,
                                              const float* bc, int r, float u, float z) {
  float acc = 0.0f;
#pragma unroll
  for (int j = 0; j < RB; ++j)
    if (j < r) acc = __builtin_fmaf(dt_in[j], p.wdt(j), acc);
  const float dt = softplus<M>(acc + p.bdt());
  const float* Bv = bc;
  const float* Cv = bc + DS;
  float y = 0.0f;
  if constexpr (scan_fused_update<DS, M>()) {
    const float dtu = dt * u;
#pragma unroll
    for (int n = 0; n < DS; ++n) {
      const float dA = exp2_neg_sel<M>(p.na(n) * dt);
      h[n] = __builtin_fmaf(dA, h[n], Bv[n] * dtu);
      y = __builtin_fmaf(h[n], Cv[n], y);
    }
  } else {
#pragma unroll
    for (int n = 0; n < DS; ++n) {
      const float dA = exp2_neg_sel<M>(p.na(n) * dt);
      const float dB = dt * Bv[n];
      h[n] = dA * h[n] + dB * u;
      y = y + h[n] * Cv[n];
    }
  }
  y = y + p.dd() * u;
  float sg = rcp_sel<M>(1.0f + exp_sel<M>(-z));
  return y * (z * sg);
}
template <int DS, int RB>
struct ScanRegs {
  const ScanCtx<DS, RB>& c;
  __device__ __forceinline__ float wdt(int j) const { return c.wdt[j]; }
  __device__ __forceinline__ float na(int n) const { return c.na[n]; }
  __device__ __forceinline__ float bdt() const { return c.bdt; }
  __device__ __forceinline__ float dd() const { return c.dd; }
};
// Scan parameters of 16 channels in shared memory, in the quad layout of
// the decode step's na_q / wdt_q (float f of quad k of channel cl at
// (k 16 + cl) 4 + f), then b_dt and D of the 16 channels: scan_lds_floats
// floats a 16-channel block.
template <int DS, int RB>
constexpr int scan_lds_floats() { return (DS + RB) * 16 + 32; }
template <int DS, int RB>
struct ScanLds {
  const float* p;
  int cl;
  __device__ __forceinline__ float na(int n) const { return p[((n >> 2) * 16 + cl) * 4 + (n & 3)]; }
  __device__ __forceinline__ float wdt(int j) const {
    return p[DS * 16 + ((j >> 2) * 16 + cl) * 4 + (j & 3)];
  }
  __device__ __forceinline__ float bdt() const { return p[(DS + RB) * 16 + cl]; }
  __device__ __forceinline__ float dd() const { return p[(DS + RB) * 16 + 16 + cl]; }
};
// Source of float4 k (< scan_lds_floats / 4) of 16-channel block c16's
// parameters in that layout.
template <int DS, int RB>
__device__ __forceinline__ const float4* scan_lds_src(const LayerW& Lw, const float* na_q,
                                                      const float* wdt_q, int c16, int k) {
  if (k < DS * 4) return reinterpret_cast<const float4*>(na_q) + (size_t)c16 * (DS / 4) * 16 + k;
  if (k < (DS + RB) * 4)
    return reinterpret_cast<const float4*>(wdt_q) + (size_t)c16 * (RB / 4) * 16 + (k - DS * 4);
  const int j = k - (DS + RB) * 4;  // 0-3 b_dt, 4-7 D
  return reinterpret_cast<const float4*>((j < 4 ? Lw.b_dt : Lw.dd) + 16 * c16) + (j & 3);
}
template <int DS, int RB, int M = MATH_BF>
__device__ __forceinline__ float scan_token(ScanCtx<DS, RB>& sc, const float* dt_in,
                                            const float* bc, int r, float u, float z) {
  return scan_token_p<DS, RB, M>(sc.h, ScanRegs<DS, RB>{sc}, dt_in, bc, r, u, z);
}

}  // namespace boa
