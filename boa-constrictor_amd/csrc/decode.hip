// Decode-step kernels (one token per lane, M = lanes rows).
//
// A decode step is a chain of small GEMMs (M = lanes ~ 10^3) plus per-lane
// recurrent state updates.  Every activation of the step, and every decode
// weight matrix, is stored k-blocked: element (feature k, lane m) at
//   ((k / 16) * ld + m) * 16 + 4 * (k % 4) + (k % 16) / 4
// (dblk below).  At MFMA k-step s, lane (i, g) of v_mfma_f32_16x16x4f32
// needs feature 4s + g; the four k-steps 4q..4q+3 therefore sit in one
// float4 of the lane, and the 16 lanes of a row group read one contiguous
// 64-byte segment.  So:
//   - a GEMM wave streams its fragments straight from L2 with one float4
//     load per operand per four MFMAs, issued two groups ahead, with no LDS
//     and no barriers (the vector memory pipeline, not the loads' latency,
//     bounded the feature-per-load form);
//   - LayerNorm stages 16 lanes' rows (64 contiguous bytes per lane and
//     block) in LDS;
//   - the scan runs 16 consecutive threads on the 16 channels of one lane
//     and loads whole feature blocks and state rows as float4.
// The per-element operation sequences are those of the chunk kernels
// (boa_math.h, mamba.hip), and every GEMM output is the same K-ordered fma
// chain, so decode logits are bit-identical to the compress logits.
#include "block_device.h"
#include "boa_kernels.h"
#include "coder_device.h"

namespace boa {

typedef float floatx4 __attribute__((ext_vector_type(4)));

// ------------------------------------------------------------------- GEMM
// A wave computes TN x TM MFMA tiles of 16 output features x 16 lanes.  Lane
// (i = lane & 15, g = lane >> 4) loads, per 16-k block q, the float4s at
// W[q][n0+16tn+i][4g..4g+3] and X[q][m0+16tm+i][4g..4g+3] (k-blocked), whose
// component e is its operand for k-step 4q+e; every accumulator sees k in
// order 0, 1, 2, ... (one fma chain per output).  Accumulator v of lane
// (i, g) holds tile row 4g+v for lane m0+16tm+i.  For k-blocked outputs the
// weights' tile rows are stored permuted (row j holds feature dperm(j) of
// its 16-row tile), so row 4g+v is feature 4v+g and lands at in-block
// position 4g+v: each lane stores one float4.  Row-major outputs (the
// logits) use unpermuted weights: row 4g+v is feature 4g+v.
// Epilogue operands that do not depend on the GEMM (bias, residual), loaded
// before the K loop so that their latency hides behind it.
// With CONV, in_proj's conv-step operands too: the lane's conv state rows,
// taps and biases of its four features.
template <bool CONV = false>
struct EpiPre {
  float b[4];
  float4 r;
  float4 cs[CONV ? 4 : 1], cw[CONV ? 4 : 1];
  float cb[CONV ? 4 : 1];
};

// SC: the conv state's cache policy at compile time (1 cached, 0 streamed)
// or -1 for a.state_cached; BIAS: a.bias is known to be set.  A runtime
// choice between two loads, or a load and a constant, joins in a register
// copy that the compiler guards with s_waitcnt vmcnt(0), which also waits
// for every load and copy issued before (the LayerNorm GEMM's weight rows).
template <bool CONV = false, int SC = -1, bool BIAS = false>
__device__ __forceinline__ void dec_epi_prefetch(const DecGemmArgs& a, int n0, int m, int g,
                                                 EpiPre<CONV>& p) {
  if (m >= a.M || n0 >= a.N) return;
#pragma unroll
  for (int e = 0; e < 4; ++e) {
    const int nf = a.row_major ? n0 + 4 * g + e : n0 + 4 * e + g;
    p.b[e] = (BIAS || a.bias) ? a.bias[min(nf, a.N - 1)] : 0.0f;
  }
  if (a.res && !a.row_major && !(a.conv_di > 0))
    p.r = reinterpret_cast<const float4*>(a.res)[((size_t)(n0 >> 4) * a.ldr + m) * 4 + g];
  if (CONV && a.conv_di > 0 && n0 < a.conv_di) {
#pragma unroll
    for (int e = 0; e < 4; ++e) {
      const int n = n0 + 4 * e + g;
      const float4* sp = reinterpret_cast<const float4*>(a.conv_state) + (size_t)n * a.ld_state + m;
      p.cs[e] = SC < 0 ? state_ld4(sp, a.state_cached) : state_ld3<SC == 1>(sp);
      p.cw[e] = reinterpret_cast<const float4*>(a.conv_w)[n];
      p.cb[e] = a.conv_b[n];
    }
  }
}

template <bool CONV = false>
__device__ __forceinline__ void dec_epilogue_impl(const DecGemmArgs& a, const floatx4 acc, int n0,
                                                  int m, int g, const EpiPre<CONV> pv, bool have) {
  const EpiPre<CONV>* pre = have ? &pv : nullptr;
  if (m >= a.M || n0 >= a.N) return;
  int nf[4];
#pragma unroll
  for (int e = 0; e < 4; ++e) nf[e] = a.row_major ? n0 + 4 * g + e : n0 + 4 * e + g;
  float v[4];
#pragma unroll
  for (int e = 0; e < 4; ++e) {
    const int n = min(nf[e], a.N - 1);
    float r = acc[e] + (pre ? pre->b[e] : (a.bias ? a.bias[n] : 0.0f));
    if (a.act == ACT_GELU) r = gelu<MATH_BR>(r);
    else if (a.act == ACT_RELU) r = fmaxf(0.0f, r);
    v[e] = r;
  }
  if (a.row_major) {
    const int nb = n0 + 4 * g;
    if (nb + 4 <= a.N) {
      *reinterpret_cast<float4*>(a.C + (size_t)m * a.ldc + nb) = make_float4(v[0], v[1], v[2], v[3]);
    } else {
#pragma unroll
      for (int e = 0; e < 4; ++e)
        if (nb + e < a.N) a.C[(size_t)m * a.ldc + nb + e] = v[e];
    }
    return;
  }
  if (a.conv_di > 0 && n0 < a.conv_di) {
    // every load of the four channels before the first state store, so that
    // they are in flight together (a store may alias a later load)
    float4 s0[4], wv[4];
    float bc[4];
#pragma unroll
    for (int e = 0; e < 4; ++e) {
      const int n = nf[e];
      const float4* st = reinterpret_cast<const float4*>(a.conv_state) + (size_t)n * a.ld_state + m;
      s0[e] = (CONV && pre) ? pre->cs[e] : state_ld4(st, a.state_cached);
      wv[e] = (CONV && pre) ? pre->cw[e] : reinterpret_cast<const float4*>(a.conv_w)[n];
      bc[e] = (CONV && pre) ? pre->cb[e] : a.conv_b[n];
    }
    float cv[4];
#pragma unroll
    for (int e = 0; e < 4; ++e) {
      float4* st = reinterpret_cast<float4*>(a.conv_state) + (size_t)nf[e] * a.ld_state + m;
      cv[e] = conv_step_value<MATH_BR>(bc[e], s0[e], v[e], wv[e]);
      state_st4(st, make_float4(s0[e].y, s0[e].z, s0[e].w, v[e]), a.state_cached);
    }
    float* o = a.conv_out + ((size_t)(n0 >> 4) * a.ldc + m) * 16 + 4 * g;
    *reinterpret_cast<float4*>(o) = make_float4(cv[0], cv[1], cv[2], cv[3]);
    return;
  }
  const int row0 = a.conv_di > 0 ? n0 - a.conv_di : n0;
  float* o = a.C + ((size_t)(row0 >> 4) * a.ldc + m) * 16 + 4 * g;
  if (a.res) {
    const float4 rv = pre ? pre->r
        : *reinterpret_cast<const float4*>(a.res + ((size_t)(n0 >> 4) * a.ldr + m) * 16 + 4 * g);
    v[0] = v[0] + rv.x; v[1] = v[1] + rv.y; v[2] = v[2] + rv.z; v[3] = v[3] + rv.w;
  }
  if (n0 + 16 <= a.N) {
    *reinterpret_cast<float4*>(o) = make_float4(v[0], v[1], v[2], v[3]);
  } else {
#pragma unroll
    for (int e = 0; e < 4; ++e)
      if (nf[e] < a.N) o[e] = v[e];
  }
}

// The epilogue operands come prefetched (pre) or are loaded here (no pre);
// the prefetched struct is passed by value so that it stays in registers.
template <bool CONV = false>
__device__ __forceinline__ void dec_epilogue(const DecGemmArgs& a, const floatx4 acc, int n0, int m,
                                             int g, const EpiPre<CONV>& pre) {
  dec_epilogue_impl<CONV>(a, acc, n0, m, g, pre, true);
}
__device__ __forceinline__ void dec_epilogue(const DecGemmArgs& a, const floatx4 acc, int n0, int m,
                                             int g) {
  dec_epilogue_impl<false>(a, acc, n0, m, g, EpiPre<false>{}, false);
}

// The K loop of one wave: loads run PD groups of UQ 16-k blocks ahead of the
// MFMAs through a ring of PD + 1 register groups (fully unrolled, so every
// ring index is a compile-time register).
template <int KS, int TM, int TN, int UQ, int PD>
__device__ __forceinline__ void dec_mainloop(const DecGemmArgs& a, int n0, int m0, int i, int g,
                                             floatx4 (&acc)[TM][TN]) {
  constexpr int QB = KS / 4;  // 16-k blocks in K
  constexpr int G = QB / UQ;  // groups of UQ blocks
  constexpr int R = (PD < G ? PD : G - 1) + 1;  // ring size
  static_assert(QB % UQ == 0, "K must be a multiple of 16 UQ");
  const float4* wp[TN];
  const float4* xp[TM];
#pragma unroll
  for (int t = 0; t < TN; ++t)
    wp[t] = reinterpret_cast<const float4*>(a.W) + (size_t)min(n0 + 16 * t + i, a.ldw - 1) * 4 + g;
#pragma unroll
  for (int t = 0; t < TM; ++t)
    xp[t] = reinterpret_cast<const float4*>(a.Xt) + (size_t)min(m0 + 16 * t + i, a.M - 1) * 4 + g;
  const size_t wq = (size_t)a.ldw * 4, xq = (size_t)a.ldx * 4;  // float4s per 16-k block
#pragma unroll
  for (int tm = 0; tm < TM; ++tm)
#pragma unroll
    for (int tn = 0; tn < TN; ++tn) acc[tm][tn] = floatx4{0.f, 0.f, 0.f, 0.f};
  float4 af[R][UQ][TN], bf[R][UQ][TM];
#define BOA_DEC_LOAD(BUF, Q0)                                                     \
  _Pragma("unroll") for (int q = 0; q < UQ; ++q) {                                \
    _Pragma("unroll") for (int t = 0; t < TN; ++t) af[BUF][q][t] = wp[t][(size_t)((Q0) + q) * wq]; \
    _Pragma("unroll") for (int t = 0; t < TM; ++t) bf[BUF][q][t] = xp[t][(size_t)((Q0) + q) * xq]; \
  }                                                                               \
  __builtin_amdgcn_sched_barrier(0);
#pragma unroll
  for (int p = 0; p < R - 1; ++p) { BOA_DEC_LOAD(p, p * UQ) }
#pragma unroll
  for (int gi = 0; gi < G; ++gi) {
    if (gi + R - 1 < G) { BOA_DEC_LOAD((gi + R - 1) % R, (gi + R - 1) * UQ) }
#pragma unroll
    for (int q = 0; q < UQ; ++q) {
#pragma unroll
      for (int e = 0; e < 4; ++e)
#pragma unroll
        for (int tm = 0; tm < TM; ++tm)
#pragma unroll
          for (int tn = 0; tn < TN; ++tn)
            acc[tm][tn] = __builtin_amdgcn_mfma_f32_16x16x4f32(af[gi % R][q][tn][e],
                                                              bf[gi % R][q][tm][e], acc[tm][tn],
                                                              0, 0, 0);
    }
    __builtin_amdgcn_sched_barrier(0);
  }
#undef BOA_DEC_LOAD
}

// One 16 x 16 tile per wave: wave w (0-3) of virtual block vb takes 16-lane
// tile w of the 64-lane group and n tile j of xcd_slot(vb, n_tiles).  Its
// bias and residual load ahead of the K loop.  No barriers.
template <int KS, int UQ, int PD>
__device__ __forceinline__ void dec_gemm_wave(const DecGemmArgs& a, int vb, int tid) {
  const int lane = tid & 63, w = tid >> 6;
  const int i = lane & 15, g = lane >> 4;
  const XcdSlot q = xcd_slot(vb, (a.N + 15) / 16);
  const int m0 = q.grp * 64 + 16 * w, n0 = q.j * 16;
  if (m0 >= a.M) return;
  EpiPre<> pre;
  dec_epi_prefetch<false>(a, n0, m0 + i, g, pre);
  floatx4 acc[1][1];
  dec_mainloop<KS, 1, 1, UQ, PD>(a, n0, m0, i, g, acc);
  dec_epilogue(a, acc[0][0], n0, m0 + i, g, pre);
}

template <int KS, int TM, int TN, int UQ, int PD>
__global__ __launch_bounds__(256) void dec_gemm_kernel(DecGemmArgs a) {
  const int lane = threadIdx.x & 63;
  const int i = lane & 15, g = lane >> 4;
  const int n_tiles = (a.N + 16 * TN - 1) / (16 * TN);
  floatx4 acc[TM][TN];
  if (TM == 1 && TN == 1) {
    // one tile per wave; a block's 4 waves take the 4 16-lane tiles of one
    // 64-lane group (xcd_slot) and one n tile
    dec_gemm_wave<KS, UQ, PD>(a, blockIdx.x, threadIdx.x);
    return;
  }
  const int m_tiles = (a.M + 16 * TM - 1) / (16 * TM);
  const int wid = blockIdx.x * (blockDim.x >> 6) + (threadIdx.x >> 6);
  if (wid >= n_tiles * m_tiles) return;  // whole waves exit; no barriers below
  const int n0 = (wid % n_tiles) * 16 * TN;
  const int m0 = (wid / n_tiles) * 16 * TM;
  dec_mainloop<KS, TM, TN, UQ, PD>(a, n0, m0, i, g, acc);
#pragma unroll
  for (int tm = 0; tm < TM; ++tm)
#pragma unroll
    for (int tn = 0; tn < TN; ++tn) dec_epilogue(a, acc[tm][tn], n0 + 16 * tn, m0 + 16 * tm + i, g);
}

// One 16 x 16 tile per wave with the weight fragments shared in LDS.  The
// block's four waves take the four 16-lane tiles of a 64-lane group and one
// 16-feature n tile, as in dec_gemm_wave, so they need the same weight
// fragment at every 16-k block.  Per stage of four 16-k blocks, wave w
// copies weight block 4 s + w (1 KB: lane i + 16 g gets the float4 of
// feature n0 + i, k quad g) straight into LDS (global_load_lds), and its own
// four activation blocks likewise; every wave then reads its operands from
// LDS, one 16-byte read per lane and block.  A CU issues 20 vector-memory
// loads per stage instead of 32: a 16-byte-per-lane load occupies the
// texture-address unit for about 32 cycles, which bounded dec_gemm_wave on
// the 1000-lane K >= 512 shapes (FF2 9.5 us against a 256-MFMA chain of
// about 6 us).  The activations go through LDS too so that every operand
// wait is this kernel's own (vm_wait): the compiler waits for all copies in
// flight (vmcnt(0)) before a register load's use once a copy to LDS is
// pending.  Same K-ordered chain, same bits.
template <int KS, int P>
__global__ __launch_bounds__(256) void dec_gemm_sw_kernel(DecGemmArgs a) {
  constexpr int QB = KS / 4, ST = QB / 4, R = P + 1;  // 16-k blocks, stages, ring slots
  static_assert(QB % 4 == 0 && ST > P, "whole stages of four 16-k blocks");
  // slot: 4 weight blocks, then 4 activation blocks of each wave
  __shared__ __align__(16) lds_u32x4 sm[R][4 + 16][64];
  const int tid = threadIdx.x, lane = tid & 63, w = tid >> 6;
  const int i = lane & 15, g = lane >> 4;
  const XcdSlot sl = xcd_slot(blockIdx.x, (a.N + 15) / 16);
  const int m0 = sl.grp * 64 + 16 * w, n0 = sl.j * 16;
  if (sl.grp * 64 >= a.M) return;  // the whole block; waves past M take part in the barriers
  EpiPre<> pre;
  dec_epi_prefetch<false>(a, n0, m0 + i, g, pre);
  const size_t wq = (size_t)a.ldw * 4, xq = (size_t)a.ldx * 4;  // float4s per 16-k block
  const lds_u32x4* wsrc = reinterpret_cast<const lds_u32x4*>(a.W) + (size_t)(n0 + i) * 4 + g + w * wq;
  const lds_u32x4* xsrc =
      reinterpret_cast<const lds_u32x4*>(a.Xt) + (size_t)min(m0 + i, a.M - 1) * 4 + g;
  auto issue = [&](int s) {  // stage s: one weight copy and four activation copies
    __builtin_amdgcn_global_load_lds((const void*)(wsrc + (size_t)(4 * s) * wq),
                                     (__attribute__((address_space(3))) void*)&sm[s % R][w][0],
                                     16, 0, 0);
#pragma unroll
    for (int u = 0; u < 4; ++u)
      __builtin_amdgcn_global_load_lds(
          (const void*)(xsrc + (size_t)(4 * s + u) * xq),
          (__attribute__((address_space(3))) void*)&sm[s % R][4 + 4 * w + u][0], 16, 0, 0);
  };
  floatx4 acc = floatx4{0.f, 0.f, 0.f, 0.f};
#pragma unroll
  for (int s = 0; s < P; ++s) issue(s);
#pragma unroll
  for (int s = 0; s < ST; ++s) {
    // this wave's copies of stage s are done (the younger stages' five
    // copies each may still run); after the barrier every wave's are in LDS
    // and every wave is done reading slot (s - 1) % R, which the copies of
    // stage s + P overwrite
    vm_wait(5 * min(P - 1, ST - 1 - s));
    lds_barrier();
    if (s + P < ST) issue(s + P);
    lds_u32x4 wf[4], xf[4];
#pragma unroll
    for (int u = 0; u < 4; ++u) {
      wf[u] = lds_read128(&sm[s % R][u][lane]);
      xf[u] = lds_read128(&sm[s % R][4 + 4 * w + u][lane]);
    }
    lds_wait8(wf[0], wf[1], wf[2], wf[3], xf[0], xf[1], xf[2], xf[3]);
#pragma unroll
    for (int u = 0; u < 4; ++u) {
      const floatx4 wv = __builtin_bit_cast(floatx4, wf[u]);
      const floatx4 xv = __builtin_bit_cast(floatx4, xf[u]);
#pragma unroll
      for (int e = 0; e < 4; ++e) acc = __builtin_amdgcn_mfma_f32_16x16x4f32(wv[e], xv[e], acc, 0, 0, 0);
    }
  }
  dec_epilogue(a, acc, n0, m0 + i, g, pre);
}

namespace {
template <int TM, int TN, int UQ, int PD>
hipError_t dec_launch(const DecGemmArgs& a, hipStream_t s) {
  const int tiles = ((a.N + 16 * TN - 1) / (16 * TN)) * ((a.M + 16 * TM - 1) / (16 * TM));
  const dim3 grid(TM == 1 && TN == 1 ? xcd_grid(a.M, (a.N + 15) / 16) : (tiles + 3) / 4), block(256);
  switch (a.K) {
    case 64: BOA_LAUNCH((dec_gemm_kernel<16, TM, TN, UQ, PD>), grid, block, 0, s, a); break;
    case 80: BOA_LAUNCH((dec_gemm_kernel<20, TM, TN, UQ, PD>), grid, block, 0, s, a); break;
    case 160: BOA_LAUNCH((dec_gemm_kernel<40, TM, TN, UQ, PD>), grid, block, 0, s, a); break;
    case 320: BOA_LAUNCH((dec_gemm_kernel<80, TM, TN, UQ, PD>), grid, block, 0, s, a); break;
    case 128: BOA_LAUNCH((dec_gemm_kernel<32, TM, TN, UQ, PD>), grid, block, 0, s, a); break;
    case 256: BOA_LAUNCH((dec_gemm_kernel<64, TM, TN, UQ, PD>), grid, block, 0, s, a); break;
    case 512: BOA_LAUNCH((dec_gemm_kernel<128, TM, TN, UQ, PD>), grid, block, 0, s, a); break;
    case 1024: BOA_LAUNCH((dec_gemm_kernel<256, TM, TN, UQ, PD>), grid, block, 0, s, a); break;
    case 2048: BOA_LAUNCH((dec_gemm_kernel<512, TM, TN, UQ, PD>), grid, block, 0, s, a); break;
    default: return hipErrorInvalidValue;  // K = d, 2d or 4d of a supported d_model
  }
  return hipGetLastError();
}

hipError_t dec_check(const DecGemmArgs& a) {
  if (a.ldw < (a.N + 15) / 16 * 16 || a.ldx < a.M || a.ldc < (a.row_major ? a.N : a.M) ||
      (a.res && a.ldr < a.M) || (a.conv_di % 16))
    return hipErrorInvalidValue;
  return hipSuccess;
}

template <int P>
hipError_t dec_launch_sw(const DecGemmArgs& a, hipStream_t s) {
  const dim3 grid(xcd_grid(a.M, (a.N + 15) / 16)), block(256);
  switch (a.K) {
    case 256: BOA_LAUNCH((dec_gemm_sw_kernel<64, P>), grid, block, 0, s, a); break;
    case 512: BOA_LAUNCH((dec_gemm_sw_kernel<128, P>), grid, block, 0, s, a); break;
    case 1024: BOA_LAUNCH((dec_gemm_sw_kernel<256, P>), grid, block, 0, s, a); break;
    case 2048: BOA_LAUNCH((dec_gemm_sw_kernel<512, P>), grid, block, 0, s, a); break;
    default: return hipErrorInvalidValue;
  }
  return hipGetLastError();
}
}  // namespace

hipError_t dec_gemm_cfg(const DecGemmArgs& a, int cfg, hipStream_t s) {
  if (a.M <= 0 || a.N <= 0) return hipSuccess;
  if (hipError_t e = dec_check(a)) return e;
  switch (cfg) {
    case 15: return dec_launch_sw<3>(a, s);
    case 4: return dec_launch<1, 1, 1, 8>(a, s);
    case 9: return dec_launch<2, 2, 1, 6>(a, s);
    case 10: return dec_launch<1, 1, 1, 2>(a, s);
    case 13: return dec_launch<4, 1, 1, 4>(a, s);
    default: return hipErrorInvalidValue;
  }
}

// Wave tiles by shape, from a sweep on MI355X (all configurations give the
// same bits): K = 256 x N >= 1024 (in_proj, FF1) runs fastest on the smallest
// register ring; from 2048 lanes on, 32 x 32 tiles halve the operand loads of
// the K >= 512 projections and 64-lane tiles those of the heads; below 2048
// lanes the other K >= 256 shapes (out_proj, FF2, the heads) share their
// weight fragments through LDS (at 1000 lanes 127 -> 110 us of these GEMMs
// per decode step, three stages in flight; two measured 0.5 us slower).
// At 4096 lanes the shared-weight form was slower for FF1 and for out_proj
// and FF2 (decode GEMMs 991 -> 1014 and 1006 us per step).
hipError_t dec_gemm(const DecGemmArgs& a, hipStream_t s) {
  int cfg = 4;
  if (a.K <= 256 && a.N >= 1024) cfg = 10;
  else if (a.M >= 2048 && a.N >= 256) cfg = a.K >= 512 ? 9 : 13;
  else if (a.M < 2048 && (a.K == 256 || a.K == 512 || a.K == 1024 || a.K == 2048)) cfg = 15;
  return dec_gemm_cfg(a, cfg, s);
}

// ----------------------------------------- head.2 fused with the decode step
// dec_head_step_kernel: head.2 (the 256 logits of a lane, no bias, K = d),
// the CDF (head.2's bias added, temperature), the symbol search and the
// coder advance in one launch, so the logits never leave the CU
// (boa_gpu.hpp:1049-1052 followed by range_coder_kernels.cu:504-627).  A
// block of 1024 threads owns 16 lanes: wave w computes logits 16w .. 16w+15
// of the 16 lanes as dec_gemm_kernel's wave does (the same K-ordered fma
// chain, + 0 as its bias-free epilogue) into LDS; then half-wave h of waves
// 0-7 runs decode_step_kernel's work for lane h.  Same bits as
// dec_gemm (head.2) + decode_step_kernel.
// LDS of the fused head step: 16 logits rows of HS_LS floats, then the 16
// CDFs (doubles) and coder targets
constexpr int HS_LS = 256 + 4;
template <int KS>
__device__ __forceinline__ void dec_head_step_body(
    const DecGemmArgs& a, const float* __restrict__ head_b2, float inv_t, uint8_t* tok,
    const int32_t* __restrict__ lens, int t, uint8_t* out, int64_t out_stride, RcDec* states,
    const uint32_t* __restrict__ payload, const uint64_t* __restrict__ offsets_words,
    const int32_t* __restrict__ sizes_words, int m0, float* lg, double (*s_cdf)[260],
    uint32_t* s_target, int tid) {
  constexpr int LS = HS_LS;  // LDS logits row stride
  if (m0 >= a.M) return;  // the whole block, before any barrier
  const int wv = tid >> 6, lane = tid & 63, i = lane & 15, g = lane >> 4;
  {
    floatx4 acc[1][1];
    dec_mainloop<KS, 1, 1, 1, 8>(a, 16 * wv, m0, i, g, acc);
#pragma unroll
    for (int v = 0; v < 4; ++v) lg[i * LS + 16 * wv + 4 * g + v] = acc[0][0][v] + 0.0f;
  }
  __syncthreads();
  const int h = tid >> 5, l = tid & 31;  // half-waves 0-15 (waves 0-7) own lanes m0 + h
  const int b = m0 + h;
  const bool mine = h < 16;
  const bool active = mine && b < a.M && t < lens[b < a.M ? b : a.M - 1];
  RcDec st;
  if (mine) {
    double r[8];
    cdf_halfwave_regs(lg + h * LS, head_b2, inv_t, l, r);
#pragma unroll
    for (int e = 0; e < 8; ++e) s_cdf[h][8 * l + e] = r[e];
    if (l == 31) s_cdf[h][256] = 1.0;
    if (active && l == 0) {
      st = states[b];
      s_target[h] = dec_target(st);
    }
  }
  __syncthreads();
  if (!active) return;  // no barrier follows
  int sym;
  uint32_t low_s, high_s;
  cdf_search_halfwave(s_cdf[h], s_target[h], l, sym, low_s, high_s);
  if (l == 0) {
    dec_advance(st, low_s, high_s, payload + offsets_words[b], sizes_words[b]);
    states[b] = st;
    out[(size_t)b * out_stride + t] = (uint8_t)sym;
    tok[b] = (uint8_t)sym;
  }
}

template <int KS>
__global__ __launch_bounds__(1024) void dec_head_step_kernel(
    DecGemmArgs a, const float* __restrict__ head_b2, float inv_t, uint8_t* tok,
    const int32_t* __restrict__ lens, const int* __restrict__ t_counter, uint8_t* out,
    int64_t out_stride, RcDec* states, const uint32_t* __restrict__ payload,
    const uint64_t* __restrict__ offsets_words, const int32_t* __restrict__ sizes_words) {
  __shared__ __align__(16) float lg[16 * HS_LS];
  __shared__ double s_cdf[16][260];
  __shared__ uint32_t s_target[16];
  const XcdSlot blk = xcd_slot(blockIdx.x, 4);  // 4 16-lane tiles per 64-lane group
  dec_head_step_body<KS>(a, head_b2, inv_t, tok, lens, *t_counter, out, out_stride, states,
                                payload, offsets_words, sizes_words, blk.grp * 64 + blk.j * 16, lg,
                                s_cdf, s_target, threadIdx.x);
}

hipError_t launch_dec_head_step(const DecGemmArgs& a, const float* head_b2, float inv_temp,
                                uint8_t* tok, const int32_t* lens, const int* t_counter,
                                uint8_t* out, int64_t out_stride, RcDec* st,
                                const uint32_t* payload, const uint64_t* offsets_words,
                                const int32_t* sizes_words, hipStream_t s) {
  if (a.M <= 0) return hipSuccess;
  if (a.N != 256 || a.ldw < 256 || a.ldx < a.M || a.row_major != 1 || a.bias)
    return hipErrorInvalidValue;
  const dim3 grid(xcd_grid(a.M, 4)), block(1024);
#define BOA_HEADSTEP(KSv)                                                                     \
  BOA_LAUNCH((dec_head_step_kernel<KSv>), grid, block, 0, s, a, head_b2, inv_temp, tok, \
                     lens, t_counter, out, out_stride, st, payload, offsets_words, sizes_words)
  switch (a.K) {
    case 64: BOA_HEADSTEP(16); break;
    case 80: BOA_HEADSTEP(20); break;
    case 128: BOA_HEADSTEP(32); break;
    case 256: BOA_HEADSTEP(64); break;
    case 512: BOA_HEADSTEP(128); break;
    default: return hipErrorInvalidValue;
  }
#undef BOA_HEADSTEP
  return hipGetLastError();
}

// ------------------------------------------------ LayerNorm + GEMM (K = d)
// in_proj (after LN1) and FF1 (after LN2) take the normalised d features of
// a lane as their whole K.  A block of 1024 threads owns 64 lanes x 64 output
// features:
//   1. it copies the 64 lanes' k-blocked rows (through registers) and the
//      64 weight rows (straight from global memory) into LDS, per 16-k block
//      one contiguous 4 KB span each, and loads the epilogue's operands;
//   2. it computes each lane's mean and rstd in the LayerNorm's reduction
//      order (dec_ln_kernel) and normalises the rows in LDS with the same
//      operations, so the operands are the bits the LayerNorm would store;
//   3. each of the 16 waves runs one 16 x 16 tile from LDS, k in the order
//      of dec_mainloop (one fma chain per output, the same bits);
//   4. the epilogue is dec_epilogue (conv step, activation, stores).
// Against LayerNorm + dec_gemm this removes a launch and the normalised
// rows' round trip through memory, and the block's waves share their
// operand loads.  Layer 0's LN1 gathers the embedding rows and the n-block
// 0 blocks store them as x.
// The block's work for virtual block vb, with its LDS passed in: xs and ws
// of NB * 1024 floats each, lwb of 2 d, stats of 128.
template <int MODE, int NB, bool EMB, int SC>
__device__ __forceinline__ void dec_ln_gemm_body(const DecGemmArgs& a, const float* __restrict__ emb,
                                                 const uint8_t* __restrict__ tok, float* xt,
                                                 const float* __restrict__ lw,
                                                 const float* __restrict__ lb, int vb, float* xs,
                                                 float* ws, float* lwb, float* stats, int tid) {
  constexpr int d = NB * 16;
  const int n = a.ln_n;               // the LayerNorm's width: features n .. d-1 are zero
  constexpr int SQ = NB / 4;          // staged float4s per thread and operand
  static_assert(NB % 4 == 0, "d must be a multiple of 64");
  const XcdSlot blk = xcd_slot(vb, a.N / 64);
  const int m0 = blk.grp * 64, n0 = blk.j * 64;
  if (m0 >= a.M) return;  // the whole block, before any barrier

  // 1. stage weights, LayerNorm parameters and rows: float4 r = tid % 256 of
  // 16-k block q = 4 it + tid / 256 (row r / 4, quarter r % 4)
  const int r = tid & 255, ml = r >> 2, a4 = r & 3;
  const int m = min(m0 + ml, a.M - 1);  // rows past M are normalised, never stored
  stream_f4 xr[SQ];  // a vector type: an array of float4 structs went through scratch
  const float4* W4 = reinterpret_cast<const float4*>(a.W);
  const float* erow = EMB ? emb + (size_t)tok[m] * d : nullptr;
#pragma unroll
  for (int it = 0; it < SQ; ++it) {
    const int q = 4 * it + (tid >> 8);
    xr[it] = EMB ? *reinterpret_cast<const stream_f4*>(erow + 16 * q + 4 * a4)
                 : reinterpret_cast<const stream_f4*>(a.Xt)[((size_t)q * a.ldx + m) * 4 + a4];
  }
  static_assert(d <= 1024, "one LayerNorm parameter per thread");
  const int kp = min(tid, d - 1);
  const float lwv = lw[kp], lbv = lb[kp];
  // threads past d store parameter d - 1 again (the same value, no branch)
  lwb[kp] = lwv;
  lwb[d + kp] = lbv;
#pragma unroll
  for (int it = 0; it < SQ; ++it) {
    const int q = 4 * it + (tid >> 8);
    float* row = xs + (q * 64 + ml) * 16;
    if (EMB) {  // natural feature order in, k-blocked positions out
      const float e4[4] = {xr[it].x, xr[it].y, xr[it].z, xr[it].w};
#pragma unroll
      for (int e = 0; e < 4; ++e) row[dperm(4 * a4 + e)] = e4[e];
    } else {
      reinterpret_cast<stream_f4*>(row)[a4] = xr[it];
    }
  }
  // the weight rows go straight to LDS (global_load_lds_dwordx4: a wave's 64
  // float4s are one contiguous 1 KB span at both ends), issued after the
  // rows' LDS stores (the scheduling barrier keeps them there): 13.4 ->
  // 13.2 us at 1000 lanes against register staging.  The compiler waits for
  // every copy before the LayerNorm's first LDS read, so they and the
  // epilogue loads below complete before step 2; staging the weights through
  // registers instead, which lets the LayerNorm run under the loads,
  // measured slower (LN GEMMs 206 -> 209.5 us per step at 1000 lanes).
  __builtin_amdgcn_sched_barrier(0);
#pragma unroll
  for (int it = 0; it < SQ; ++it) {
    const int q = 4 * it + (tid >> 8);
    __builtin_amdgcn_global_load_lds(
        (const void*)(W4 + ((size_t)q * a.ldw + n0) * 4 + r),
        (__attribute__((address_space(3))) void*)(reinterpret_cast<float4*>(ws) + q * 256 + (r & ~63)),
        16, 0, 0);
  }
  // LDS barrier without the fence of __syncthreads, which would wait for the
  // weight copies too: this wave's LDS stores are complete at lgkmcnt(0)
  asm volatile("s_waitcnt lgkmcnt(0)\n\ts_barrier" ::: "memory");
  // the epilogue's operands (bias, and in_proj's conv state, taps and
  // biases), loaded now so that their latency hides behind the LayerNorm
  // and the MFMAs; the row loads above have been waited for
  const int lane_ = tid & 63, wv_ = tid >> 6;
  const int lr_ = 16 * (wv_ >> 2) + (lane_ & 15), fn0 = n0 + 16 * (wv_ & 3);
  EpiPre<MODE == 1> pre;
  dec_epi_prefetch<MODE == 1, SC, true>(a, fn0, m0 + lr_, lane_ >> 4, pre);
  if (EMB && n0 == 0 && m0 + ml < a.M) {  // layer 0: x = embedding rows
#pragma unroll
    for (int it = 0; it < SQ; ++it) {
      const int q = 4 * it + (tid >> 8);
      reinterpret_cast<float4*>(xt)[((size_t)q * a.ldx + m0 + ml) * 4 + a4] =
          reinterpret_cast<const float4*>(xs + (q * 64 + ml) * 16)[a4];
    }
  }

  // 2. statistics (the orders of dec_ln_kernel) and normalisation
  if (MODE == 1) {
    const int lj = tid >> 4, l = tid & 15;
    auto xat = [xs, lj](int f) { return xs[((f >> 4) * 64 + lj) * 16 + dperm(f & 15)]; };
    float s0 = 0.0f, q0 = 0.0f, s1 = 0.0f, q1 = 0.0f;
#pragma unroll
    for (int f = l; f < d; f += 32) {
      const float x = xat(f);
      s0 = s0 + x;
      q0 = q0 + x * x;
    }
#pragma unroll
    for (int f = l + 16; f < d; f += 32) {
      const float x = xat(f);
      s1 = s1 + x;
      q1 = q1 + x * x;
    }
    float sum = s0 + s1, sq = q0 + q1;
#pragma unroll
    for (int off = 8; off > 0; off >>= 1) {
      sum = sum + __shfl_down(sum, off, 16);
      sq = sq + __shfl_down(sq, off, 16);
    }
    if (l == 0) {
      const float mean = sum / (float)n;
      const float var = sq / (float)n - mean * mean;
      stats[2 * lj] = mean;
      stats[2 * lj + 1] = 1.0f / __builtin_sqrtf(var + 1e-5f);
    }
  } else if (tid < 128) {  // LN2: lane tid % 64's sum (wave 0) and sum of squares (wave 1)
    const int lj = tid & 63;
    const bool squares = tid >= 64;
    float acc = 0.0f;
#pragma unroll 2
    for (int q = 0; q < NB; ++q) {
      const float4* row = reinterpret_cast<const float4*>(xs + (q * 64 + lj) * 16);
      const float4 c0 = row[0], c1 = row[1], c2 = row[2], c3 = row[3];
      // position p holds feature dperm(p): features 16q + 0, 1, 2, ... sit at
      // positions 0, 4, 8, 12, 1, 5, ...
      const float fv[16] = {c0.x, c1.x, c2.x, c3.x, c0.y, c1.y, c2.y, c3.y,
                            c0.z, c1.z, c2.z, c3.z, c0.w, c1.w, c2.w, c3.w};
#pragma unroll
      for (int j = 0; j < 16; ++j) acc = acc + (squares ? fv[j] * fv[j] : fv[j]);
    }
    stats[2 * lj + (squares ? 1 : 0)] = acc;
  }
  asm volatile("s_waitcnt lgkmcnt(0)\n\ts_barrier" ::: "memory");
  {
    float mean, rstd;
    if (MODE == 1) {
      mean = stats[2 * ml];
      rstd = stats[2 * ml + 1];
    } else {  // from the two sums, as dec_ln_kernel
      mean = stats[2 * ml] / (float)n;
      const float var = stats[2 * ml + 1] / (float)n - mean * mean;
      rstd = 1.0f / __builtin_sqrtf(var + 1e-5f);
    }
#pragma unroll
    for (int it = 0; it < SQ; ++it) {
      const int q = 4 * it + (tid >> 8);
      float4* p4 = reinterpret_cast<float4*>(xs + (q * 64 + ml) * 16) + a4;
      const float4 v = *p4;
      const float x[4] = {v.x, v.y, v.z, v.w};
      float o[4];
#pragma unroll
      for (int e = 0; e < 4; ++e) {
        const int f = 16 * q + dperm(4 * a4 + e);
        o[e] = ((x[e] - mean) * rstd) * lwb[f] + lwb[d + f];
      }
      *p4 = make_float4(o[0], o[1], o[2], o[3]);
    }
  }
  __builtin_amdgcn_s_waitcnt(0);  // this wave's weight rows have reached LDS
  __syncthreads();

  // 3. MFMAs from LDS: wave w runs the 16 x 16 tile of lanes 16 (w / 4) + i,
  // features 16 (w % 4) + i
  const int lane = tid & 63, wv = tid >> 6;
  const int i = lane & 15, g = lane >> 4;
  const int lr = 16 * (wv >> 2) + i, fr = 16 * (wv & 3) + i;
  floatx4 acc = floatx4{0.f, 0.f, 0.f, 0.f};
#pragma unroll
  for (int q = 0; q < NB; ++q) {
    const float4 bv = reinterpret_cast<const float4*>(xs + (q * 64 + lr) * 16)[g];
    const float4 av = reinterpret_cast<const float4*>(ws + (q * 64 + fr) * 16)[g];
    acc = __builtin_amdgcn_mfma_f32_16x16x4f32(av.x, bv.x, acc, 0, 0, 0);
    acc = __builtin_amdgcn_mfma_f32_16x16x4f32(av.y, bv.y, acc, 0, 0, 0);
    acc = __builtin_amdgcn_mfma_f32_16x16x4f32(av.z, bv.z, acc, 0, 0, 0);
    acc = __builtin_amdgcn_mfma_f32_16x16x4f32(av.w, bv.w, acc, 0, 0, 0);
  }
  // 4. epilogue
  dec_epilogue<MODE == 1>(a, acc, n0 + 16 * (wv & 3), m0 + lr, g, pre);
}

// SC: the conv state's cache policy (in_proj; 0 for FF1)
template <int MODE, int NB, bool EMB, int SC>
__global__ __launch_bounds__(1024) void dec_ln_gemm_kernel(DecGemmArgs a, const float* __restrict__ emb,
                                                           const uint8_t* __restrict__ tok, float* xt,
                                                           const float* __restrict__ lw,
                                                           const float* __restrict__ lb,
                                                           int* t_counter) {
  constexpr int TILE = NB * 64 * 16;  // floats of a 64-row k-blocked tile
  __shared__ __align__(16) float xs[TILE];
  __shared__ __align__(16) float ws[TILE];
  __shared__ float lwb[2 * NB * 16];
  __shared__ float stats[2 * 64];
  if (t_counter && blockIdx.x == 0 && threadIdx.x == 0) *t_counter += 1;
  dec_ln_gemm_body<MODE, NB, EMB, SC>(a, emb, tok, xt, lw, lb, blockIdx.x, xs, ws, lwb, stats,
                                      threadIdx.x);
}

bool dec_ln_gemm_fits(int d, int N) { return (d == 64 || d == 128 || d == 256) && N % 64 == 0; }

hipError_t launch_dec_ln_gemm(int mode, const DecGemmArgs& a, const float* emb, const uint8_t* tok,
                              float* xt, const float* lw, const float* lb, int* t_counter,
                              hipStream_t s) {
  if (a.M <= 0) return hipSuccess;
  if (!dec_ln_gemm_fits(a.K, a.N) || (mode != 1 && mode != 2) || (emb && mode != 1) || !a.bias ||
      a.ldw < a.N || a.ldx < a.M || a.ldc < (a.row_major ? a.N : a.M) ||
      (a.res && a.ldr < a.M) || (a.conv_di % 16))
    return hipErrorInvalidValue;
  const dim3 grid(xcd_grid(a.M, a.N / 64)), block(1024);
#define BOA_LNG(NBv)                                                                          \
  if (emb && a.state_cached)                                                                  \
    BOA_LAUNCH((dec_ln_gemm_kernel<1, NBv, true, 1>), grid, block, 0, s, a, emb, tok, xt, \
               lw, lb, t_counter);                                                            \
  else if (emb)                                                                               \
    BOA_LAUNCH((dec_ln_gemm_kernel<1, NBv, true, 0>), grid, block, 0, s, a, emb, tok, xt, \
               lw, lb, t_counter);                                                            \
  else if (mode == 1 && a.state_cached)                                                       \
    BOA_LAUNCH((dec_ln_gemm_kernel<1, NBv, false, 1>), grid, block, 0, s, a, emb, tok, xt, \
               lw, lb, t_counter);                                                            \
  else if (mode == 1)                                                                         \
    BOA_LAUNCH((dec_ln_gemm_kernel<1, NBv, false, 0>), grid, block, 0, s, a, emb, tok, xt, \
               lw, lb, t_counter);                                                            \
  else                                                                                        \
    BOA_LAUNCH((dec_ln_gemm_kernel<2, NBv, false, 0>), grid, block, 0, s, a, emb, tok, xt, \
               lw, lb, t_counter);
  switch (a.K) {
    case 64: BOA_LNG(4) break;
    case 128: BOA_LNG(8) break;
    case 256: BOA_LNG(16) break;
    default: return hipErrorInvalidValue;
  }
#undef BOA_LNG
  return hipGetLastError();
}

// Weight relayout for decode: W [K][ldw_in] row-major (the compress layout)
// -> k-blocked [K/16][ldn][16].  Logical output column j maps to source
// column j (j < zs), to a zero column (zs <= j < ze) or to source column
// j - (ze - zs) (j >= ze); with `permute`, tile row j of every 16-row
// output tile holds logical column (j & ~15) + dperm(j & 15) (dperm is its
// own inverse).
__global__ void dec_weight_blk_kernel(const float* __restrict__ w, int ldw_in, int n_src,
                                      float* out, int K, int ldn, int permute, int zs, int ze) {
  const size_t idx = (size_t)blockIdx.x * blockDim.x + threadIdx.x;
  if (idx >= (size_t)K * ldn) return;
  const int k = (int)(idx / ldn), j = (int)(idx % ldn);
  const int jl = permute ? (j & ~15) + dperm(j & 15) : j;
  const int n = jl < zs ? jl : (jl < ze ? -1 : jl - (ze - zs));
  out[dblk(k, j, ldn)] = (n >= 0 && n < n_src) ? w[(size_t)k * ldw_in + n] : 0.0f;
}

hipError_t launch_dec_weight_blk(const float* w, int ldw_in, int n_src, float* out, int K, int ldn,
                                 int permute, int zs, int ze, hipStream_t s) {
  if (K % 16 || ldn % 16 || n_src > ldw_in || zs > ze) return hipErrorInvalidValue;
  const size_t n = (size_t)K * ldn;
  BOA_LAUNCH(dec_weight_blk_kernel, dim3((unsigned)((n + 255) / 256)), dim3(256), 0, s, w,
                     ldw_in, n_src, out, K, ldn, permute, zs, ze);
  return hipGetLastError();
}

// Per-channel scan parameters in the decode scan's quad layout: element
// (c, j) of a [di][n] table at (((c/16) n/4 + j/4) 16 + c%16) 4 + j%4.
// dt_proj weights come from [r][di] (zero padded to rb), -exp(A_log) log2(e) from
// [di][ds].
__device__ __forceinline__ size_t quad_idx(int c, int j, int n) {
  return ((size_t)((c >> 4) * (n >> 2) + (j >> 2)) * 16 + (c & 15)) * 4 + (j & 3);
}

__global__ void dec_scan_params_kernel(const float* __restrict__ w_dt, const float* __restrict__ na,
                                       float* wdt_q, float* na_q, int r, int rb, int ds, int di) {
  const int idx = blockIdx.x * blockDim.x + threadIdx.x;
  if (idx < di * rb) {
    const int c = idx / rb, j = idx % rb;
    wdt_q[quad_idx(c, j, rb)] = j < r ? w_dt[(size_t)j * di + c] : 0.0f;
  }
  if (idx < di * ds) {
    const int c = idx / ds, n = idx % ds;
    na_q[quad_idx(c, n, ds)] = na[idx];
  }
}

hipError_t launch_dec_scan_params(const float* w_dt, const float* na, float* wdt_q, float* na_q,
                                  int r, int rb, int ds, int di, hipStream_t s) {
  if (di % 16 || rb % 4 || ds % 4) return hipErrorInvalidValue;
  const int n = di * (rb > ds ? rb : ds);
  BOA_LAUNCH(dec_scan_params_kernel, dim3((n + 255) / 256), dim3(256), 0, s, w_dt, na, wdt_q,
                     na_q, r, rb, ds, di);
  return hipGetLastError();
}

// -------------------------------------------------------------- LayerNorm
// A block of 16 LANES threads normalises LANES lanes.  Thread t loads
// float4 t % 4 of lane t / 4 % LANES's feature block t / (4 LANES) + 4 it
// (a wavefront reads 64 LANES contiguous bytes per feature block), the slab
// is kept in LDS in natural feature order, the statistics follow the
// reference's order, and each thread normalises and stores the float4s it
// loaded.  Small blocks spread the 1000-odd lanes of a decode step over
// more CUs.
//   LN1 (MODE 1): 16 threads per lane; thread l sums features l, l+32, ...
//     and l+16, l+48, ... (the partials of lanes l and l+16 of the
//     reference's warp-per-row reduction), adds them (the shuffle step 16)
//     and finishes the shuffle-down tree 8, 4, 2, 1 -- the order of the
//     compress LN1 kernel.
//   LN2 (MODE 2): one thread per lane sums all features in order.
// Layer 0's LN1 reads the embedding rows instead (and stores them as x).
constexpr int DEC_LN_LANES = 4;

template <int MODE, int NB, bool EMB, int LANES>
__global__ __launch_bounds__(16 * LANES) void dec_ln_kernel(const float* __restrict__ emb,
                                                     const uint8_t* __restrict__ tok, float* xt,
                                                     const float* src, float* xnt,
                                                     const float* __restrict__ w,
                                                     const float* __restrict__ b, int M, int ld,
                                                     int* t_counter, int n) {
  constexpr int d = NB * 16;
  constexpr int S = d + 4;                 // LDS row stride (floats)
  constexpr int IT = (NB + 3) / 4;         // feature blocks per thread
  __shared__ __align__(16) float tile[LANES * S];
  __shared__ float stats[2 * LANES];
  if (t_counter && blockIdx.x == 0 && threadIdx.x == 0) *t_counter += 1;
  const int t = threadIdx.x;
  const int j = (t >> 2) % LANES, a4 = t & 3, kb0 = t / (4 * LANES);
  const int m0 = blockIdx.x * LANES;
  const int m = min(m0 + j, M - 1);
  const float* erow = EMB ? emb + (size_t)tok[m] * d : nullptr;
  float4 v[IT];
#pragma unroll
  for (int it = 0; it < IT; ++it) {
    const int kb = kb0 + 4 * it;
    if (kb < NB) {
      v[it] = EMB ? *reinterpret_cast<const float4*>(erow + 16 * kb + 4 * a4)
                  : *reinterpret_cast<const float4*>(src + ((size_t)kb * ld + m) * 16 + 4 * a4);
    }
  }
#pragma unroll
  for (int it = 0; it < IT; ++it) {
    const int kb = kb0 + 4 * it;
    if (kb < NB) {
      float* row = tile + j * S + 16 * kb;
      const float e4[4] = {v[it].x, v[it].y, v[it].z, v[it].w};
#pragma unroll
      for (int e = 0; e < 4; ++e) row[EMB ? 4 * a4 + e : dperm(4 * a4 + e)] = e4[e];
    }
  }
  __syncthreads();
  if (MODE == 1) {
    const int lj = t >> 4, l = t & 15;
    const float* row = tile + lj * S;
    float s0 = 0.0f, q0 = 0.0f, s1 = 0.0f, q1 = 0.0f;
#pragma unroll 4
    for (int k = l; k < d; k += 32) {
      const float x = row[k];
      s0 = s0 + x;
      q0 = q0 + x * x;
    }
#pragma unroll 4
    for (int k = l + 16; k < d; k += 32) {
      const float x = row[k];
      s1 = s1 + x;
      q1 = q1 + x * x;
    }
    float sum = s0 + s1, sq = q0 + q1;
#pragma unroll
    for (int off = 8; off > 0; off >>= 1) {
      sum = sum + __shfl_down(sum, off, 16);
      sq = sq + __shfl_down(sq, off, 16);
    }
    if (l == 0) {
      const float mean = sum / (float)n;
      const float var = sq / (float)n - mean * mean;
      stats[2 * lj] = mean;
      stats[2 * lj + 1] = 1.0f / __builtin_sqrtf(var + 1e-5f);
    }
  } else if (t < LANES) {
    const float4* row = reinterpret_cast<const float4*>(tile + t * S);
    float sum = 0.0f, sq = 0.0f;
#pragma unroll 8
    for (int k4 = 0; k4 < d / 4; ++k4) {
      const float4 x = row[k4];
      sum = sum + x.x; sq = sq + x.x * x.x;
      sum = sum + x.y; sq = sq + x.y * x.y;
      sum = sum + x.z; sq = sq + x.z * x.z;
      sum = sum + x.w; sq = sq + x.w * x.w;
    }
    const float mean = sum / (float)n;
    const float var = sq / (float)n - mean * mean;
    stats[2 * t] = mean;
    stats[2 * t + 1] = 1.0f / __builtin_sqrtf(var + 1e-5f);
  }
  __syncthreads();
  if (m0 + j >= M) return;
  const float mean = stats[2 * j], rstd = stats[2 * j + 1];
#pragma unroll
  for (int it = 0; it < IT; ++it) {
    const int kb = kb0 + 4 * it;
    if (kb < NB) {
      const float* row = tile + j * S + 16 * kb;
      float x[4], o[4];
#pragma unroll
      for (int e = 0; e < 4; ++e) {
        const int f = dperm(4 * a4 + e);  // feature in block at position 4 a4 + e
        x[e] = row[f];
        o[e] = ((x[e] - mean) * rstd) * w[16 * kb + f] + b[16 * kb + f];
      }
      const size_t off = ((size_t)kb * ld + m0 + j) * 16 + 4 * a4;
      if (EMB) *reinterpret_cast<float4*>(xt + off) = make_float4(x[0], x[1], x[2], x[3]);
      *reinterpret_cast<float4*>(xnt + off) = make_float4(o[0], o[1], o[2], o[3]);
    }
  }
}

namespace {
template <int MODE>
hipError_t dec_ln_launch(const float* emb, const uint8_t* tok, float* xt, const float* src,
                         float* xnt, const float* w, const float* b, int M, int d, int n, int ld,
                         int* t_counter, hipStream_t s) {
  constexpr int LN = DEC_LN_LANES;
  const dim3 grid((M + LN - 1) / LN), block(16 * LN);
#define BOA_DEC_LN(NBv)                                                                      \
  if (emb)                                                                                   \
    BOA_LAUNCH((dec_ln_kernel<MODE, NBv, true, LN>), grid, block, 0, s, emb, tok, xt, \
                       src, xnt, w, b, M, ld, t_counter, n);                                 \
  else                                                                                       \
    BOA_LAUNCH((dec_ln_kernel<MODE, NBv, false, LN>), grid, block, 0, s, emb, tok,   \
                       xt, src, xnt, w, b, M, ld, t_counter, n);
  switch (d) {
    case 64: BOA_DEC_LN(4) break;
    case 80: BOA_DEC_LN(5) break;
    case 128: BOA_DEC_LN(8) break;
    case 256: BOA_DEC_LN(16) break;
    case 512: BOA_DEC_LN(32) break;
    default: return hipErrorInvalidValue;  // decode needs d_model in {64, 80, 128, 256, 512}
  }
#undef BOA_DEC_LN
  return hipGetLastError();
}
}  // namespace

hipError_t launch_dec_ln1(const float* emb, const uint8_t* tok, float* xt, float* xnt,
                          const float* w, const float* b, int M, int d, int n, int ld,
                          int* t_counter, hipStream_t s) {
  return dec_ln_launch<1>(emb, tok, xt, xt, xnt, w, b, M, d, n, ld, t_counter, s);
}

hipError_t launch_dec_ln2(const float* xt, float* xnt, const float* w, const float* b, int M, int d,
                          int n, int ld, hipStream_t s) {
  return dec_ln_launch<2>(nullptr, nullptr, nullptr, xt, xnt, w, b, M, d, n, ld, nullptr, s);
}

// ------------------------------------------------------------------- scan
// Thread t of block (x, y): channel c = 16 y + t % 16, lane m = 16 x + t / 16.
// The decode x_proj writes its row with dt_in at features [0, r), zeros up
// to RB, B at [RB, RB + DS) and C at [RB + DS, RB + 2 DS), so the thread
// loads whole 16-feature blocks (float4) and indexes them at compile time.
// State, -exp(A_log) log2(e) and dt_proj weights are stored in quads of four n (or j)
// with the 16 channels of a channel block innermost, so that every float4
// load of a wavefront reads one contiguous 1 KB (state) or 256 B span:
//   h[c][n] of lane m at ((((c/16) DS/4 + n/4) ld_state + m) 16 + c%16) 4 + n%4
//   na[c][n]          at (((c/16) DS/4 + n/4) 16 + c%16) 4 + n%4
//   wdt[c][j]         at (((c/16) RB/4 + j/4) 16 + c%16) 4 + j%4
template <int DS, int RB, bool CACHED>
__global__ __launch_bounds__(256) void dec_scan_kernel(LayerW Lw, const float* __restrict__ na_q,
                                                       const float* __restrict__ wdt_q,
                                                       const float* __restrict__ zt,
                                                       const float* __restrict__ cvt,
                                                       const float* __restrict__ rows,
                                                       float* ssm, float* yt, int M, int ld,
                                                       int ld_state, int r, int cbn) {
  constexpr int NB = (RB + 2 * DS + 15) / 16;
  // the block's 16 lanes' x_proj rows (NB k-blocked 16-feature blocks each),
  // loaded once and read by the 16 channel threads of each lane
  __shared__ __align__(16) float4 srow[16 * NB * 4];
  const int cl = threadIdx.x & 15;
  const XcdSlot blk = xcd_slot(blockIdx.x, 4 * cbn);  // cbn channel blocks x 4 16-lane blocks
  const int cb = blk.j % cbn;
  const int c = cb * 16 + cl;
  const int m0 = blk.grp * 64 + (blk.j / cbn) * 16;
  if (m0 >= M) return;  // the whole block, before the barrier
  for (int q = threadIdx.x; q < 16 * NB * 4; q += 256) {
    const int lm = q / (NB * 4), kb = (q / 4) % NB, c4 = q % 4;
    const int mq = min(m0 + lm, M - 1);
    srow[q] = reinterpret_cast<const float4*>(rows)[((size_t)kb * ld + mq) * 4 + c4];
  }
  __syncthreads();
  const int lm = threadIdx.x >> 4;
  const int m = m0 + lm;
  if (m >= M) return;  // after the block's only barrier
  ScanCtx<DS, RB> sc;
  float4* h4 = reinterpret_cast<float4*>(ssm);
  const float4* na4 = reinterpret_cast<const float4*>(na_q);
  const float4* w4 = reinterpret_cast<const float4*>(wdt_q);
#pragma unroll
  for (int n4 = 0; n4 < DS / 4; ++n4) {
    const float4 hv =
        state_ld4(h4 + ((size_t)(cb * (DS / 4) + n4) * ld_state + m) * 16 + cl, CACHED);
    sc.h[4 * n4] = hv.x; sc.h[4 * n4 + 1] = hv.y; sc.h[4 * n4 + 2] = hv.z; sc.h[4 * n4 + 3] = hv.w;
    const float4 av = na4[(cb * (DS / 4) + n4) * 16 + cl];
    sc.na[4 * n4] = av.x; sc.na[4 * n4 + 1] = av.y; sc.na[4 * n4 + 2] = av.z; sc.na[4 * n4 + 3] = av.w;
  }
#pragma unroll
  for (int j4 = 0; j4 < RB / 4; ++j4) {
    const float4 wv = w4[(cb * (RB / 4) + j4) * 16 + cl];
    sc.wdt[4 * j4] = wv.x; sc.wdt[4 * j4 + 1] = wv.y; sc.wdt[4 * j4 + 2] = wv.z; sc.wdt[4 * j4 + 3] = wv.w;
  }
  sc.bdt = Lw.b_dt[c];
  sc.dd = Lw.dd[c];
  float row[NB * 16];
#pragma unroll
  for (int kb = 0; kb < NB; ++kb) {
    float f[16];
#pragma unroll
    for (int a4 = 0; a4 < 4; ++a4) {
      const float4 t = srow[(lm * NB + kb) * 4 + a4];
      f[4 * a4] = t.x; f[4 * a4 + 1] = t.y; f[4 * a4 + 2] = t.z; f[4 * a4 + 3] = t.w;
    }
#pragma unroll
    for (int j = 0; j < 16; ++j) row[16 * kb + j] = f[dperm(j)];
  }
  const size_t cm = dblk(c, m, ld);
  const float u = cvt[cm];
  const float z = zt[cm];
  yt[cm] = scan_token<DS, RB, MATH_BR>(sc, row, row + RB, r, u, z);
#pragma unroll
  for (int n4 = 0; n4 < DS / 4; ++n4)
    state_st4(h4 + ((size_t)(cb * (DS / 4) + n4) * ld_state + m) * 16 + cl,
              make_float4(sc.h[4 * n4], sc.h[4 * n4 + 1], sc.h[4 * n4 + 2], sc.h[4 * n4 + 3]), CACHED);
}

// ------------------------------------------------ x_proj fused with the scan
// dec_xscan_kernel runs x_proj and the scan of one layer in one launch.  A
// block of 1024 threads owns 16 lanes x 128 channels:
//   1. waves 0 .. NB-1 each run one 16-feature block of the lanes' x_proj
//      row (dt_in, B, C; K = di) as dec_gemm_kernel's wave does -- the same
//      K-ordered fma chain, then + 0 as the bias-free epilogue -- and store
//      it to LDS in natural feature order (position 4g + v of a lane's
//      float4 is feature 4v + g of its block), then issue the loads of
//      their threads' SSM state, conv output and z;
//   2. meanwhile the other waves copy the block's scan parameters to LDS and
//      issue the same loads for their threads;
//   3. after the block's only barrier, each thread runs the scan of its lane
//      for two channels (c and c + 64) in turn, reading dt_in, B and C and
//      the parameters from LDS (the 16 channel threads of a lane read the
//      same row words, the 16 lanes of a channel the same parameters).
// x_proj is recomputed by the di / 128 blocks of a 16-lane tile (4 at
// d_model 256) instead of being stored and reloaded, which removes a launch
// and the rows' round trip per layer; the bits are those of dec_gemm +
// dec_scan_kernel.  d_state 16 and d_model <= 256 only (larger shapes keep
// the two kernels: their state, decay and dt_proj registers do not fit
// 1024 threads).
// LDS floats of the x_proj rows of dec_xscan_body
template <int DS, int RB>
constexpr int xscan_lds_floats() { return 16 * (((RB + 2 * DS + 15) / 16) * 16 + 4); }

// Thread tid's lane and channels in virtual block vb of the x_proj + scan:
// lane m0 + lm (loads clamp it to mc), channel 16 (8 cb + q + 4 p) + cl of
// channel pass p = 0, 1.
template <int DI>
struct XscanPos {
  int cb, m0, cl, lm, q, m, mc;
  __device__ __forceinline__ XscanPos(int vb, int tid, int M) {
    const XcdSlot blk = xcd_slot(vb, 4 * (DI / 128));  // 4 16-lane tiles x DI/128 channel blocks
    cb = blk.j % (DI / 128);
    m0 = blk.grp * 64 + (blk.j / (DI / 128)) * 16;
    cl = tid & 15; lm = (tid >> 4) & 15; q = tid >> 8;
    m = m0 + lm;
    mc = min(m, M - 1);  // lanes past M load a valid row and store nothing
  }
};

// A thread's state of both channels (loaded ahead of the scan).
template <int DS, int RB>
struct XscanPre {
  float h0[DS], h1[DS];
};
template <int DS, int RB, int DI, bool CACHED>
__device__ __forceinline__ void xscan_load_state(XscanPre<DS, RB>& pr, const XscanPos<DI>& ps,
                                                 const float* ssm, int ld_state) {
  const float4* h4 = reinterpret_cast<const float4*>(ssm);
#pragma unroll
  for (int n4 = 0; n4 < DS / 4; ++n4) {
    const float4 hv = state_ld4(
        h4 + ((size_t)((8 * ps.cb + ps.q) * (DS / 4) + n4) * ld_state + ps.mc) * 16 + ps.cl, CACHED);
    pr.h0[4 * n4] = hv.x; pr.h0[4 * n4 + 1] = hv.y; pr.h0[4 * n4 + 2] = hv.z; pr.h0[4 * n4 + 3] = hv.w;
  }
#pragma unroll
  for (int n4 = 0; n4 < DS / 4; ++n4) {
    const float4 hv = state_ld4(
        h4 + ((size_t)((8 * ps.cb + ps.q + 4) * (DS / 4) + n4) * ld_state + ps.mc) * 16 + ps.cl,
        CACHED);
    pr.h1[4 * n4] = hv.x; pr.h1[4 * n4 + 1] = hv.y; pr.h1[4 * n4 + 2] = hv.z; pr.h1[4 * n4 + 3] = hv.w;
  }
}
// The block's work for virtual block vb, its x_proj rows in LDS at rown and
// its 128 channels' scan parameters at par (eight 16-channel blocks of
// scan_lds_floats); pl holds a thread's state.
template <int DS, int RB, int DI, bool CACHED>
__device__ __forceinline__ void dec_xscan_body(const LayerW& Lw, const float* __restrict__ na_q,
                                               const float* __restrict__ wdt_q,
                                               const float* __restrict__ w_x, int ldw_x,
                                               const float* __restrict__ zt,
                                               const float* __restrict__ cvt, float* ssm, float* yt,
                                               int M, int ld, int ld_state, int r, int vb,
                                               float* rown, float* par, int tid,
                                               XscanPre<DS, RB>& pl) {
  constexpr int NB = (RB + 2 * DS + 15) / 16;  // 16-feature blocks of the x_proj row
  constexpr int RS = NB * 16 + 4;              // LDS row stride (floats, 16-byte aligned)
  static_assert(NB <= 16 && DI % 128 == 0, "one wave per x_proj feature block");
  const XscanPos<DI> ps(vb, tid, M);
  const int cb = ps.cb, m0 = ps.m0, cl = ps.cl, lm = ps.lm, q = ps.q, m = ps.m, mc = ps.mc;
  if (m0 >= M) return;  // the whole block, before the barrier
  float4* h4 = reinterpret_cast<float4*>(ssm);
  const int wv = tid >> 6;
  // 1. both channels' state (16-channel blocks 8 cb + q and 8 cb + q + 4)
  // and their conv output and z (of lane mc).  The waves that run x_proj
  // issue them after it: the vector memory counter completes in order, so
  // an x_proj operand load issued behind them would wait for the state's
  // HBM round trip (18.2 us per launch at 1000 lanes with the second
  // channel's state loaded after the first channel's scan, 16.6 with both
  // before x_proj, 16.1 with the x_proj waves' own after it).
  float uz[2][2];
  auto load_scan_operands = [&]() {
    xscan_load_state<DS, RB, DI, CACHED>(pl, ps, ssm, ld_state);
#pragma unroll
    for (int p = 0; p < 2; ++p) {
      const size_t cmp = dblk(16 * (8 * cb + q + 4 * p) + cl, mc, ld);
      uz[p][0] = cvt[cmp];
      uz[p][1] = zt[cmp];
    }
  };
  // 2. x_proj: wave w < NB computes feature block w for lanes m0 .. m0 + 15
  if (wv < NB) {
    const int lane = tid & 63, i = lane & 15, g = lane >> 4;
    DecGemmArgs a{};
    a.Xt = cvt; a.ldx = ld; a.W = w_x; a.ldw = ldw_x; a.M = M; a.N = NB * 16; a.K = DI;
    floatx4 acc[1][1];
    dec_mainloop<DI / 4, 1, 1, 1, 4>(a, 16 * wv, m0, i, g, acc);
#pragma unroll
    for (int v = 0; v < 4; ++v)  // the bias-free epilogue of dec_gemm_kernel: acc + 0
      rown[i * RS + 16 * wv + 4 * v + g] = acc[0][0][v] + 0.0f;
    load_scan_operands();
  } else {
    // the other waves copy the block's scan parameters to LDS (through
    // registers: a copy straight to LDS makes the compiler wait for every
    // load in flight before the scan's LDS reads), loaded ahead of their
    // scan operands so that the copies' waits do not cover those (scan
    // 129 -> 123 us per decode step at 1000 lanes against each thread
    // loading its channels' parameters, the second channel's after the
    // first channel's scan)
    constexpr int S4 = scan_lds_floats<DS, RB>() / 4, TOT = 8 * S4;
    constexpr int NT = (16 - NB) * 64, PER = (TOT + NT - 1) / NT;
    static_assert(PER * NT - TOT <= TOT, "repeated copies fall in range");
    float4 v[PER];
    int at[PER];
#pragma unroll
    for (int k = 0; k < PER; ++k) {
      int t = tid - NB * 64 + NT * k;
      t = t < TOT ? t : t - TOT;
      at[k] = t;
      v[k] = *scan_lds_src<DS, RB>(Lw, na_q, wdt_q, 8 * cb + t / S4, t % S4);
    }
    load_scan_operands();
#pragma unroll
    for (int k = 0; k < PER; ++k) reinterpret_cast<float4*>(par)[at[k]] = v[k];
  }
  // the block's only barrier, without the fence of __syncthreads (which
  // would wait for every load in flight): the LDS stores are done at
  // lgkmcnt(0)
  asm volatile("s_waitcnt lgkmcnt(0)\n\ts_barrier" ::: "memory");
  if (m >= M) return;  // after the block's only barrier
  const float* row = rown + lm * RS;
  // 3. channels c and c + 64 of the lane, one after the other
#pragma unroll
  for (int p = 0; p < 2; ++p) {
    const int c16 = 8 * cb + q + 4 * p;
    const int c = 16 * c16 + cl;
    const size_t cm = dblk(c, m, ld);
    const float u = uz[p][0];
    const float z = uz[p][1];
    float h[DS];
#pragma unroll
    for (int n = 0; n < DS; ++n) h[n] = p == 0 ? pl.h0[n] : pl.h1[n];
    const ScanLds<DS, RB> sp{par + (q + 4 * p) * scan_lds_floats<DS, RB>(), cl};
    yt[cm] = scan_token_p<DS, RB, MATH_BR>(h, sp, row, row + RB, r, u, z);
#pragma unroll
    for (int n4 = 0; n4 < DS / 4; ++n4)
      state_st4(h4 + ((size_t)(c16 * (DS / 4) + n4) * ld_state + m) * 16 + cl,
                make_float4(h[4 * n4], h[4 * n4 + 1], h[4 * n4 + 2], h[4 * n4 + 3]), CACHED);
  }
}

template <int DS, int RB, int DI, bool CACHED>
__global__ __launch_bounds__(1024) void dec_xscan_kernel(LayerW Lw, const float* __restrict__ na_q,
                                                         const float* __restrict__ wdt_q,
                                                         const float* __restrict__ w_x, int ldw_x,
                                                         const float* __restrict__ zt,
                                                         const float* __restrict__ cvt,
                                                         float* ssm, float* yt, int M, int ld,
                                                         int ld_state, int r) {
  __shared__ __align__(16) float rown[xscan_lds_floats<DS, RB>()];
  __shared__ __align__(16) float par[8 * scan_lds_floats<DS, RB>()];
  XscanPre<DS, RB> pl;
  dec_xscan_body<DS, RB, DI, CACHED>(Lw, na_q, wdt_q, w_x, ldw_x, zt, cvt, ssm, yt, M, ld,
                                     ld_state, r, blockIdx.x, rown, par, threadIdx.x, pl);
}

bool dec_xscan_fits(const Dims& D) {
  const int rb = dec_rb(D.r);
  return D.ds == 16 && ((D.di == 128 && rb == 8) || (D.di == 256 && rb == 8) ||
                        (D.di == 512 && rb == 16));
}

hipError_t launch_dec_xscan(const Dims& D, const LayerW& Lw, const float* na_q, const float* wdt_q,
                            const float* w_x, int ldw_x, const float* zt, const float* cvt,
                            float* ssm, float* yt, int M, int ld, int ld_state, bool state_cached,
                            hipStream_t s) {
  if (!dec_xscan_fits(D) || ldw_x < dec_rb(D.r) + 2 * D.ds || ld < M) return hipErrorInvalidValue;
  const dim3 grid(xcd_grid(M, 4 * (D.di / 128))), block(1024);
#define BOA_XSCAN(RBv, DIv)                                                                       \
  if (state_cached)                                                                               \
    BOA_LAUNCH((dec_xscan_kernel<16, RBv, DIv, true>), grid, block, 0, s, Lw, na_q, wdt_q,  \
                       w_x, ldw_x, zt, cvt, ssm, yt, M, ld, ld_state, D.r);                        \
  else                                                                                            \
    BOA_LAUNCH((dec_xscan_kernel<16, RBv, DIv, false>), grid, block, 0, s, Lw, na_q, wdt_q, \
                       w_x, ldw_x, zt, cvt, ssm, yt, M, ld, ld_state, D.r)
  if (D.di == 128) BOA_XSCAN(8, 128);
  else if (D.di == 256) BOA_XSCAN(8, 256);
  else BOA_XSCAN(16, 512);
#undef BOA_XSCAN
  return hipGetLastError();
}

hipError_t launch_dec_scan(const Dims& D, const LayerW& Lw, const float* na_q, const float* wdt_q,
                           const float* zt, const float* cvt, const float* rows, float* ssm, float* yt,
                           int M, int ld, int ld_state, bool state_cached, hipStream_t s) {
  if (D.di % 16 || dec_rb(D.r) < D.r) return hipErrorInvalidValue;
  const dim3 grid(xcd_grid(M, 4 * (D.di / 16)));
#define BOA_DEC_SCAN(DSv, RBv)                                                                  \
  if (state_cached)                                                                             \
    BOA_LAUNCH((dec_scan_kernel<DSv, RBv, true>), grid, dim3(256), 0, s, Lw, na_q, wdt_q, \
                       zt, cvt, rows, ssm, yt, M, ld, ld_state, D.r, D.di / 16);                 \
  else                                                                                          \
    BOA_LAUNCH((dec_scan_kernel<DSv, RBv, false>), grid, dim3(256), 0, s, Lw, na_q, wdt_q,\
                       zt, cvt, rows, ssm, yt, M, ld, ld_state, D.r, D.di / 16)
  const int rb = dec_rb(D.r);
  if (D.ds == 16) {
    if (rb == 8) BOA_DEC_SCAN(16, 8);
    else if (rb == 16) BOA_DEC_SCAN(16, 16);
    else BOA_DEC_SCAN(16, 32);
  } else if (D.ds == 32) {
    if (rb == 8) BOA_DEC_SCAN(32, 8);
    else if (rb == 16) BOA_DEC_SCAN(32, 16);
    else BOA_DEC_SCAN(32, 32);
  } else {
    return hipErrorInvalidValue;
  }
#undef BOA_DEC_SCAN
  return hipGetLastError();
}

// --------------------------------------------------- state layout changes
// chunk layout: conv [lane][c][4], ssm [lane][c][n]
// step layout:  conv [c][lane][4], ssm [c/16][n/4][lane][c%16][n%4] (lane stride ld_state)
// (bf16 precision: the step-layout conv state is four bf16 per channel and
// lane, see state_ld4h)
__global__ void state_to_step_kernel(const float* conv_in, const float* ssm_in, float* conv_out,
                                     float* ssm_out, int lanes, int di, int ds, int ld_state,
                                     int conv_b16) {
  const int idx = blockIdx.x * blockDim.x + threadIdx.x;
  if (idx >= lanes * di) return;
  const int b = idx / di, c = idx % di;
  const float4 cv = reinterpret_cast<const float4*>(conv_in)[idx];
  if (conv_b16)
    reinterpret_cast<ushort4*>(conv_out)[(size_t)c * ld_state + b] =
        make_ushort4(f32_to_bf16(cv.x), f32_to_bf16(cv.y), f32_to_bf16(cv.z), f32_to_bf16(cv.w));
  else
    reinterpret_cast<float4*>(conv_out)[(size_t)c * ld_state + b] = cv;
  for (int n = 0; n < ds; ++n)
    ssm_out[((((size_t)(c >> 4) * (ds >> 2) + (n >> 2)) * ld_state + b) * 16 + (c & 15)) * 4 +
            (n & 3)] = ssm_in[(size_t)idx * ds + n];
}

__global__ void state_to_chunk_kernel(const float* conv_in, const float* ssm_in, float* conv_out,
                                      float* ssm_out, int lanes, int di, int ds, int ld_state,
                                      int conv_b16) {
  const int idx = blockIdx.x * blockDim.x + threadIdx.x;
  if (idx >= lanes * di) return;
  const int b = idx / di, c = idx % di;
  if (conv_b16) {
    const ushort4 h = reinterpret_cast<const ushort4*>(conv_in)[(size_t)c * ld_state + b];
    reinterpret_cast<float4*>(conv_out)[idx] =
        make_float4(bf16_to_f32(h.x), bf16_to_f32(h.y), bf16_to_f32(h.z), bf16_to_f32(h.w));
  } else {
    reinterpret_cast<float4*>(conv_out)[idx] =
        reinterpret_cast<const float4*>(conv_in)[(size_t)c * ld_state + b];
  }
  for (int n = 0; n < ds; ++n)
    ssm_out[(size_t)idx * ds + n] =
        ssm_in[((((size_t)(c >> 4) * (ds >> 2) + (n >> 2)) * ld_state + b) * 16 + (c & 15)) * 4 +
               (n & 3)];
}

hipError_t launch_state_relayout(const float* conv_in, const float* ssm_in, float* conv_out,
                                 float* ssm_out, int lanes, int di, int ds, int ld_state,
                                 bool to_step, bool conv_b16, hipStream_t s) {
  const int n = lanes * di;
  if (to_step)
    BOA_LAUNCH(state_to_step_kernel, dim3((n + 255) / 256), dim3(256), 0, s, conv_in,
                       ssm_in, conv_out, ssm_out, lanes, di, ds, ld_state, conv_b16 ? 1 : 0);
  else
    BOA_LAUNCH(state_to_chunk_kernel, dim3((n + 255) / 256), dim3(256), 0, s, conv_in,
                       ssm_in, conv_out, ssm_out, lanes, di, ds, ld_state, conv_b16 ? 1 : 0);
  return hipGetLastError();
}

}  // namespace boa
