// Persistent decode for small models (d_model 64): one block of 1024 threads
// owns 16 lanes and runs every decode step of a batch for them -- embedding,
// the L blocks, the head, the CDF, the symbol search and the coder advance --
// with the step's activations in LDS and no synchronisation between blocks
// (decode lanes are independent).  It replaces the step's launch chain
// (6 L + 3 kernels per step, each a few microseconds of launch and drain at
// this size) by block barriers.
//
// It covers, for one batch, what the reference's decompress loop runs per
// step as a graph replay (portability_solved_cpp/boa.cpp:672-774):
// BoaPredictorGPU::step_batch (boa_gpu.hpp:1034-1053; blocks :835-843,
// Mamba step :227-247, feed-forward :739-764, head :1049-1052) and the fused
// decode step of range_coder_kernels.cu:491-629 (CDF, symbol search, coder
// advance).
//
// Every operation is the one of the step kernels (decode.hip, coder.hip),
// with the same operand arrangement and k order in every MFMA chain, the
// same LayerNorm reduction orders and the same epilogue order (bias,
// activation, residual), so the logits, and therefore the symbols, are
// bit-identical to the launch-chain step and to the compress pass.  The
// state layouts in global memory (conv, SSM, coder, token) are those of the
// step kernels, so either path can continue where the other stopped.
#include "block_device.h"
#include "coder_device.h"

namespace boa {

namespace {

typedef float floatx4 __attribute__((ext_vector_type(4)));

constexpr int PL = 16;  // MFMA rows of the block's tiles: the lane capacity of its LDS rows

// One 16 x 16 tile of the block's 16 lanes and features n0 .. n0 + 15.  A:
// activations in LDS, k-blocked with lane capacity 16 (feature k of lane m at
// ((k / 16) 16 + m) 16 + dperm(k % 16)); W: k-blocked decode weights in
// global memory with capacity ldw.  Lane (i, g) feeds W row n0 + i and lane
// i's float4 g of every 16-k block, four MFMAs per block in k order -- the
// arrangement of dec_mainloop.
template <int KB>
__device__ __forceinline__ floatx4 pd_tile(const float* A, const float* __restrict__ W, int ldw,
                                           int n0, int i, int g) {
  const float4* w4 = reinterpret_cast<const float4*>(W) + (size_t)(n0 + i) * 4 + g;
  const size_t wq = (size_t)ldw * 4;
  constexpr int CH = KB < 8 ? KB : 8;  // weight float4s loaded ahead of their MFMAs
  floatx4 acc = floatx4{0.f, 0.f, 0.f, 0.f};
#pragma unroll
  for (int q0 = 0; q0 < KB; q0 += CH) {
    float4 wv[CH];
#pragma unroll
    for (int q = 0; q < CH; ++q) wv[q] = w4[(size_t)(q0 + q) * wq];
#pragma unroll
    for (int q = 0; q < CH; ++q) {
      const float4 bv = reinterpret_cast<const float4*>(A + ((q0 + q) * PL + i) * 16)[g];
      acc = __builtin_amdgcn_mfma_f32_16x16x4f32(wv[q].x, bv.x, acc, 0, 0, 0);
      acc = __builtin_amdgcn_mfma_f32_16x16x4f32(wv[q].y, bv.y, acc, 0, 0, 0);
      acc = __builtin_amdgcn_mfma_f32_16x16x4f32(wv[q].z, bv.z, acc, 0, 0, 0);
      acc = __builtin_amdgcn_mfma_f32_16x16x4f32(wv[q].w, bv.w, acc, 0, 0, 0);
    }
  }
  return acc;
}

// The tile's float4 for lane i: k-blocked outputs (permuted weight rows) hold
// feature n0 + 4 e + g in component e, at in-block position 4 g + e.
__device__ __forceinline__ float4* pd_out(float* base, int n0, int i, int g) {
  return reinterpret_cast<float4*>(base + ((n0 >> 4) * PL + i) * 16) + g;
}

// LayerNorm statistics of the block's 16 lanes (xs k-blocked, d features).
// MODE 1 (LN1): 16 threads per lane, the reference's warp-tree order, stats =
// (mean, rstd).  MODE 2 (LN2): sequential sums (one thread for the sum, one
// for the squares), stats = (sum, sum of squares).  The orders of
// dec_ln_gemm_kernel.  n: the LayerNorm's width (features n .. d-1 are zero).
template <int MODE, int NB>
__device__ __forceinline__ void pd_ln_stats(const float* xs, float* stats, int tid, int n) {
  constexpr int d = NB * 16;
  if (MODE == 1) {
    if (tid >= 16 * PL) return;
    const int lj = tid >> 4, l = tid & 15;
    auto xat = [&](int f) { return xs[((f >> 4) * PL + lj) * 16 + dperm(f & 15)]; };
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
  } else {
    if (tid >= 2 * PL) return;
    const int lj = tid & 15;
    const bool squares = tid >= PL;
    float acc = 0.0f;
#pragma unroll
    for (int q = 0; q < NB; ++q) {
      const float4* row = reinterpret_cast<const float4*>(xs + (q * PL + lj) * 16);
      const float4 c0 = row[0], c1 = row[1], c2 = row[2], c3 = row[3];
      // position p holds feature dperm(p): features 16 q + 0, 1, 2, ... sit
      // at positions 0, 4, 8, 12, 1, 5, ...
      const float fv[16] = {c0.x, c1.x, c2.x, c3.x, c0.y, c1.y, c2.y, c3.y,
                            c0.z, c1.z, c2.z, c3.z, c0.w, c1.w, c2.w, c3.w};
#pragma unroll
      for (int j = 0; j < 16; ++j) acc = acc + (squares ? fv[j] * fv[j] : fv[j]);
    }
    stats[2 * lj + (squares ? 1 : 0)] = acc;
  }
}

template <int MODE, int NB>
__device__ __forceinline__ void pd_ln_apply(const float* xs, float* xn, const float* stats,
                                            const float* __restrict__ w,
                                            const float* __restrict__ b, int tid, int n) {
  for (int p = tid; p < NB * 256; p += 1024) {
    const int q = p >> 8, m = (p >> 4) & 15, f = 16 * q + dperm(p & 15);
    float mean, rstd;
    if (MODE == 1) {
      mean = stats[2 * m];
      rstd = stats[2 * m + 1];
    } else {
      mean = stats[2 * m] / (float)n;
      const float var = stats[2 * m + 1] / (float)n - mean * mean;
      rstd = 1.0f / __builtin_sqrtf(var + 1e-5f);
    }
    xn[p] = ((xs[p] - mean) * rstd) * w[f] + b[f];
  }
}

}  // namespace

// LP lanes per block (16, 8 or 4): rows LP .. 15 of every MFMA tile are
// inert (an MFMA output column depends on its own row of activations only;
// their loads read a lane of this block and nothing is stored for them), so
// a block's matrix-core chains cost the same for any LP, while its VALU
// phases (the scan's 16 exponentials per channel, GELU, the CDF) scale with
// LP.  Fewer lanes per block spread those phases over more CUs.
template <int NB, int RB, int LP>
__global__ __launch_bounds__(1024) void dec_persist_kernel(PersistArgs a) {
  static_assert(LP == 4 || LP == 8 || LP == 16, "lanes per block");
  constexpr int LSH = LP == 4 ? 2 : LP == 8 ? 3 : 4;
  constexpr int d = NB * 16, DI = 2 * d, NBI = 2 * NB, NBF = 4 * NB, DS = 16;
  constexpr int NBX = (RB + 2 * DS + 15) / 16;  // 16-blocks of the x_proj row
  constexpr int RW = NBX * 16 + 1;              // LDS row stride of the x_proj rows
  __shared__ __align__(16) float xs[NB * 256];   // residual stream x
  __shared__ __align__(16) float xn[NB * 256];   // LayerNorm output
  __shared__ __align__(16) float zs[NBI * 256];  // z half of in_proj
  __shared__ __align__(16) float cvs[NBI * 256]; // conv + SiLU output
  __shared__ __align__(16) float rwn[PL * RW];   // x_proj rows (dt_in, B, C), natural order
  __shared__ __align__(16) float ys[NBI * 256];  // scan output
  __shared__ __align__(16) float os[NB * 256];   // out_proj / head1 output
  __shared__ __align__(16) float hid[NBF * 256]; // FF1 output
  __shared__ __align__(16) float lg[PL * 256];   // logits, row-major
  __shared__ double s_cdf[PL][260];
  __shared__ float stats[2 * PL];
  __shared__ int tok_s[PL];
  // per-channel parameters of every layer and the head biases, staged once
  constexpr int O_LN1W = 0, O_LN1B = O_LN1W + d, O_BIN = O_LN1B + d, O_CONVW = O_BIN + 2 * DI,
                O_CONVB = O_CONVW + 4 * DI, O_BDT = O_CONVB + DI, O_DD = O_BDT + DI,
                O_NAQ = O_DD + DI, O_WDTQ = O_NAQ + DS * DI, O_BOUT = O_WDTQ + RB * DI,
                O_LN2W = O_BOUT + d, O_LN2B = O_LN2W + d, O_B1 = O_LN2B + d, O_B2 = O_B1 + 4 * d,
                PSZ = O_B2 + d;
  __shared__ __align__(16) float prm[PERSIST_MAX_LAYERS * PSZ];
  __shared__ float hb1[d], hb2[256];
  const int tid0 = threadIdx.x;
  const int m0 = blockIdx.x * LP;
  // coder: half-wave h < 16 decodes lane m0 + h; its lane 0 holds the state
  const int half = tid0 >> 5, l = tid0 & 31;
  const int mh = m0 + half;
  const bool coder_lane = half < LP && mh < a.lanes;
  RcDec st{};
  if (coder_lane && l == 0) st = a.states[mh];
  const int len_h = coder_lane ? a.lens[mh] : 0;
  // the lane's stream, read once (the byte stores of the step loop could
  // alias these arrays, so the compiler would reload them every step) and
  // its next word loaded ahead (dec_advance_ahead)
  const uint32_t* pin = nullptr;
  int32_t pn = 0;
  uint32_t nw = 0;
  if (coder_lane && l == 0) {
    pin = a.payload + a.offsets[mh];
    pn = a.sizes[mh];
    nw = st.read_idx_words < pn ? pin[st.read_idx_words] : 0u;
  }
  if (tid0 < PL) tok_s[tid0] = tid0 < LP ? a.tok[min(m0 + tid0, a.lanes - 1)] : 0;
  auto stage = [&](float* dst, const float* __restrict__ src, int n) {
    for (int k = tid0; k < n; k += 1024) dst[k] = src[k];
  };
#pragma unroll
  for (int li = 0; li < PERSIST_MAX_LAYERS; ++li) {
    if (li >= a.L) break;
    const PersistLayer& P = a.layer[li];
    float* q = prm + li * PSZ;
    stage(q + O_LN1W, P.ln1_w, d); stage(q + O_LN1B, P.ln1_b, d);
    stage(q + O_BIN, P.b_in, 2 * DI); stage(q + O_CONVW, P.conv_w, 4 * DI);
    stage(q + O_CONVB, P.conv_b, DI); stage(q + O_BDT, P.b_dt, DI); stage(q + O_DD, P.dd, DI);
    stage(q + O_NAQ, P.na_q, DS * DI); stage(q + O_WDTQ, P.wdt_q, RB * DI);
    stage(q + O_BOUT, P.b_out, d); stage(q + O_LN2W, P.ln2_w, d); stage(q + O_LN2B, P.ln2_b, d);
    stage(q + O_B1, P.b1, 4 * d); stage(q + O_B2, P.b2, d);
  }
  stage(hb1, a.hb1, d);
  stage(hb2, a.hb2, 256);
  __syncthreads();

  for (int t = 1; t < a.maxlen; ++t) {
    // the thread index passes through an opaque move each step, so that the
    // many addresses derived from it are recomputed in the step instead of
    // being hoisted out of the loop (and spilled)
    int tid = tid0;
    asm volatile("" : "+v"(tid));
    const int wv = tid >> 6, i = tid & 15, g = (tid >> 4) & 3;
    const int mi = min(m0 + min(i, LP - 1), a.lanes - 1);  // lane of MFMA row i (state index)
    const bool mi_ok = i < LP && m0 + i < a.lanes;
#pragma unroll
    for (int li = 0; li < PERSIST_MAX_LAYERS; ++li) {  // unrolled: constant kernel-argument offsets
      if (li >= a.L) break;
      const PersistLayer& P = a.layer[li];
      const float* q = prm + li * PSZ;
      if (li == 0) {  // x = embedding rows of the current tokens
        for (int p = tid; p < NB * 256; p += 1024) {
          const int q = p >> 8, m = (p >> 4) & 15;
          xs[p] = a.emb[(size_t)tok_s[m] * d + 16 * q + dperm(p & 15)];
        }
        __syncthreads();
      }
      pd_ln_stats<1, NB>(xs, stats, tid, a.ln_n);
      __syncthreads();
      pd_ln_apply<1, NB>(xs, xn, stats, q + O_LN1W, q + O_LN1B, tid, a.ln_n);
      __syncthreads();
      // in_proj: features < DI run the conv step (state float4 [c][lane]),
      // features >= DI are z
      for (int tile = wv; tile < 2 * NBI; tile += 16) {
        const int n0 = tile * 16;
        float4 s0[4];  // conv state, loaded ahead of the MFMA chain
        if (n0 < DI) {
#pragma unroll
          for (int e = 0; e < 4; ++e)
            s0[e] = reinterpret_cast<const float4*>(P.conv)[(size_t)(n0 + 4 * e + g) * a.ld_state + mi];
        }
        const floatx4 acc = pd_tile<NB>(xn, P.w_in, 2 * DI, n0, i, g);
        float v[4];
#pragma unroll
        for (int e = 0; e < 4; ++e) v[e] = acc[e] + q[O_BIN + n0 + 4 * e + g];
        if (n0 < DI) {
          float cv[4];
#pragma unroll
          for (int e = 0; e < 4; ++e) {
            const int n = n0 + 4 * e + g;
            const float4 cw = reinterpret_cast<const float4*>(q + O_CONVW)[n];
            cv[e] = conv_step_value<MATH_BR>(q[O_CONVB + n], s0[e], v[e], cw);
            if (mi_ok)
              reinterpret_cast<float4*>(P.conv)[(size_t)n * a.ld_state + mi] =
                  make_float4(s0[e].y, s0[e].z, s0[e].w, v[e]);
          }
          *pd_out(cvs, n0, i, g) = make_float4(cv[0], cv[1], cv[2], cv[3]);
        } else {
          *pd_out(zs, n0 - DI, i, g) = make_float4(v[0], v[1], v[2], v[3]);
        }
      }
      __syncthreads();
      // x_proj (no bias: + 0 as the step's epilogue)
      for (int tile = wv; tile < NBX; tile += 16) {
        const floatx4 acc = pd_tile<NBI>(cvs, P.w_x, NBX * 16, tile * 16, i, g);
#pragma unroll
        for (int e = 0; e < 4; ++e) rwn[i * RW + tile * 16 + 4 * e + g] = acc[e] + 0.0f;
      }
      __syncthreads();
      // scan: item (lane lm, channel c), the operations of dec_scan_kernel
#pragma unroll 1
      for (int it = tid; it < LP * DI; it += 1024) {
        const int cl = it & 15, lm = (it >> 4) & (LP - 1), cb = it >> (4 + LSH);
        const int c = cb * 16 + cl;
        const int m = min(m0 + lm, a.lanes - 1);
        float4* h4 = reinterpret_cast<float4*>(P.ssm);
        const float4* na4 = reinterpret_cast<const float4*>(q + O_NAQ);
        const float4* w4 = reinterpret_cast<const float4*>(q + O_WDTQ);
        ScanCtx<DS, RB> sc;
#pragma unroll
        for (int n4 = 0; n4 < DS / 4; ++n4) {
          const float4 hv = h4[((size_t)(cb * (DS / 4) + n4) * a.ld_state + m) * 16 + cl];
          sc.h[4 * n4] = hv.x; sc.h[4 * n4 + 1] = hv.y; sc.h[4 * n4 + 2] = hv.z; sc.h[4 * n4 + 3] = hv.w;
          const float4 av = na4[(cb * (DS / 4) + n4) * 16 + cl];
          sc.na[4 * n4] = av.x; sc.na[4 * n4 + 1] = av.y; sc.na[4 * n4 + 2] = av.z; sc.na[4 * n4 + 3] = av.w;
        }
#pragma unroll
        for (int j4 = 0; j4 < RB / 4; ++j4) {
          const float4 wd = w4[(cb * (RB / 4) + j4) * 16 + cl];
          sc.wdt[4 * j4] = wd.x; sc.wdt[4 * j4 + 1] = wd.y; sc.wdt[4 * j4 + 2] = wd.z; sc.wdt[4 * j4 + 3] = wd.w;
        }
        sc.bdt = q[O_BDT + c];
        sc.dd = q[O_DD + c];
        const float* row = rwn + lm * RW;
        const int cp = ((c >> 4) * PL + lm) * 16 + dperm(c & 15);
        ys[cp] = scan_token<DS, RB, MATH_BR>(sc, row, row + RB, a.r, cvs[cp], zs[cp]);
        if (m0 + lm < a.lanes) {
#pragma unroll
          for (int n4 = 0; n4 < DS / 4; ++n4)
            h4[((size_t)(cb * (DS / 4) + n4) * a.ld_state + m) * 16 + cl] =
                make_float4(sc.h[4 * n4], sc.h[4 * n4 + 1], sc.h[4 * n4 + 2], sc.h[4 * n4 + 3]);
        }
      }
      __syncthreads();
      // out_proj + bias
      for (int tile = wv; tile < NB; tile += 16) {
        const int n0 = tile * 16;
        const floatx4 acc = pd_tile<NBI>(ys, P.w_out, d, n0, i, g);
        float v[4];
#pragma unroll
        for (int e = 0; e < 4; ++e) v[e] = acc[e] + q[O_BOUT + n0 + 4 * e + g];
        *pd_out(os, n0, i, g) = make_float4(v[0], v[1], v[2], v[3]);
      }
      __syncthreads();
      pd_ln_stats<2, NB>(os, stats, tid, a.ln_n);
      __syncthreads();
      pd_ln_apply<2, NB>(os, xn, stats, q + O_LN2W, q + O_LN2B, tid, a.ln_n);
      __syncthreads();
      // FF1 + bias + GELU
      for (int tile = wv; tile < NBF; tile += 16) {
        const int n0 = tile * 16;
        const floatx4 acc = pd_tile<NB>(xn, P.w1, 4 * d, n0, i, g);
        float v[4];
#pragma unroll
        for (int e = 0; e < 4; ++e) v[e] = gelu<MATH_BR>(acc[e] + q[O_B1 + n0 + 4 * e + g]);
        *pd_out(hid, n0, i, g) = make_float4(v[0], v[1], v[2], v[3]);
      }
      __syncthreads();
      // FF2 + bias + residual (each float4 of x read and written by one lane)
      for (int tile = wv; tile < NB; tile += 16) {
        const int n0 = tile * 16;
        const floatx4 acc = pd_tile<NBF>(hid, P.w2, d, n0, i, g);
        float4* xp = pd_out(xs, n0, i, g);
        const float4 rv = *xp;
        float v[4];
#pragma unroll
        for (int e = 0; e < 4; ++e) v[e] = acc[e] + q[O_B2 + n0 + 4 * e + g];
        *xp = make_float4(v[0] + rv.x, v[1] + rv.y, v[2] + rv.z, v[3] + rv.w);
      }
      __syncthreads();
    }
    // head1 + bias + ReLU
    for (int tile = wv; tile < NB; tile += 16) {
      const int n0 = tile * 16;
      const floatx4 acc = pd_tile<NB>(xs, a.hw1, d, n0, i, g);
      float v[4];
#pragma unroll
      for (int e = 0; e < 4; ++e) v[e] = fmaxf(0.0f, acc[e] + hb1[n0 + 4 * e + g]);
      *pd_out(os, n0, i, g) = make_float4(v[0], v[1], v[2], v[3]);
    }
    __syncthreads();
    // head2, row-major (unpermuted weights: component e is feature n0 + 4 g + e),
    // without b2 (the CDF adds it)
    for (int tile = wv; tile < 16; tile += 16) {
      const int n0 = tile * 16;
      const floatx4 acc = pd_tile<NB>(os, a.hw2, 256, n0, i, g);
      *reinterpret_cast<float4*>(lg + i * 256 + n0 + 4 * g) =
          make_float4(acc[0] + 0.0f, acc[1] + 0.0f, acc[2] + 0.0f, acc[3] + 0.0f);
    }
    __syncthreads();
    // CDF of each lane's row on its half-wave
    if (half < LP) {
      double r[8];
      cdf_halfwave_regs(lg + half * 256, hb2, a.inv_t, l, r);
#pragma unroll
      for (int k = 0; k < 8; ++k) s_cdf[half][8 * l + k] = r[k];
      if (l == 31) s_cdf[half][256] = 1.0;
    }
    __syncthreads();
    // symbol search (8 rounds of 32 candidates, ballot + first set bit) and
    // the coder advance, as decode_step_kernel
    if (coder_lane && t < len_h) {  // uniform over the half-wave
      const uint32_t target = __shfl(l == 0 ? dec_target(st) : 0u, 0, 32);
      const double* sc = s_cdf[half];
      int sym = 0;
      uint32_t low_s = 0, high_s = 0;
      const int shift = tid0 & 32;
      for (int round = 0; round < 8; ++round) {
        const int k = round * 32 + l;
        const uint32_t lo = q_low(sc, k), hi = q_high(sc, k);
        const bool match = target >= lo && target < hi;
        const uint32_t mask = (uint32_t)(__ballot(match) >> shift);
        if (mask != 0u) {
          const int winner = __ffs(mask) - 1;
          sym = __shfl(k, winner, 32);
          low_s = __shfl(lo, winner, 32);
          high_s = __shfl(hi, winner, 32);
          break;
        }
      }
      if (l == 0) {
        dec_advance_ahead(st, low_s, high_s, pin, pn, nw);
        a.out[(size_t)mh * a.out_stride + t] = (uint8_t)sym;
        tok_s[half] = sym;
      }
    }
    __syncthreads();
  }
  if (coder_lane && l == 0) {
    a.states[mh] = st;
    a.tok[mh] = (uint8_t)tok_s[half];
  }
  if (blockIdx.x == 0 && tid0 == 0) *a.t_counter = a.maxlen > 1 ? a.maxlen - 1 : 0;
}

bool dec_persist_fits(int d, int ds, int r, int L) {
  return d == 64 && ds == 16 && dec_rb(r) == 8 && L >= 1 && L <= PERSIST_MAX_LAYERS;
}

int dec_persist_lanes_per_block(int lanes, int n_cus) {
  for (int lp = 4; lp < PL; lp *= 2)
    if ((lanes + lp - 1) / lp <= n_cus) return lp;
  return PL;
}

hipError_t launch_dec_persist(const PersistArgs& a, int d, int ds, int n_cus, hipStream_t s) {
  if (a.lanes <= 0 || a.maxlen <= 1) return hipSuccess;
  if (!dec_persist_fits(d, ds, a.r, a.L)) return hipErrorInvalidValue;
  const int lp = dec_persist_lanes_per_block(a.lanes, n_cus);
  const dim3 grid((a.lanes + lp - 1) / lp), block(1024);
  if (lp == 4)
    BOA_LAUNCH((dec_persist_kernel<4, 8, 4>), grid, block, 0, s, a);
  else if (lp == 8)
    BOA_LAUNCH((dec_persist_kernel<4, 8, 8>), grid, block, 0, s, a);
  else
    BOA_LAUNCH((dec_persist_kernel<4, 8, 16>), grid, block, 0, s, a);
  return hipGetLastError();
}

}  // namespace boa
