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
//   - LayerNorm stages a 16-lane slab (contiguous in this layout) in LDS;
//   - the scan runs 16 consecutive threads on the 16 channels of one lane
//     block, so activations and the k-blocked state are read coalesced.
// The per-element operation sequences are those of the chunk kernels
// (boa_math.h, mamba.hip), and every GEMM output is the same K-ordered fma
// chain, so decode logits are bit-identical to the compress logits.
#include "block_device.h"
#include "boa_kernels.h"

namespace boa {

typedef float floatx4 __attribute__((ext_vector_type(4)));

// In-block position of feature k % 16 (a 4x4 transpose, its own inverse).
__device__ __forceinline__ int dperm(int j) { return ((j & 3) << 2) | ((j >> 2) & 3); }

// k-blocked index of (feature k, lane m), lane capacity ld.
__device__ __forceinline__ size_t dblk(int k, int m, int ld) {
  return ((size_t)(k >> 4) * ld + m) * 16 + dperm(k & 15);
}

// ------------------------------------------------------------------- GEMM
// Wave tile: 16 output features x 16 lanes.  Lane (i = lane & 15,
// g = lane >> 4) loads the float4 at W[q][n0+i][4g..4g+3] and
// X[q][m0+i][4g..4g+3] (k-blocked), whose component e is its operand for
// k-step 4q+e; the accumulated k order is 0, 1, 2, ... (one fma chain).
// Accumulator v of lane (i, g) holds tile row 4g+v for lane m0+i.  For
// k-blocked outputs the weights' tile rows are stored permuted (row j holds
// feature n0 + dperm(j)), so row 4g+v is feature n0 + 4v + g and lands at
// in-block position 4g+v: each lane stores one float4.  Row-major outputs
// (the logits) use unpermuted weights: row 4g+v is feature n0 + 4g + v.
template <int KS>
__global__ __launch_bounds__(256) void dec_gemm_kernel(DecGemmArgs a) {
  constexpr int UQ = 2;             // 16-k blocks per prefetch group
  constexpr int QB = KS / 4;        // 16-k blocks in K
  constexpr int G = QB / UQ;        // groups
  static_assert(QB % UQ == 0, "K must be a multiple of 32");
  const int lane = threadIdx.x & 63;
  const int i = lane & 15, g = lane >> 4;
  const int n_tiles = (a.N + 15) / 16;
  const int m_tiles = (a.M + 15) / 16;
  const int wid = blockIdx.x * (blockDim.x >> 6) + (threadIdx.x >> 6);
  if (wid >= n_tiles * m_tiles) return;  // whole waves exit; no barriers below
  const int n0 = (wid % n_tiles) * 16;
  const int m0 = (wid / n_tiles) * 16;
  const int mrow = min(m0 + i, a.M - 1);
  const float4* wp = reinterpret_cast<const float4*>(a.W) + (size_t)(n0 + i) * 4 + g;
  const float4* xp = reinterpret_cast<const float4*>(a.Xt) + (size_t)mrow * 4 + g;
  const size_t wq = (size_t)a.ldw * 4, xq = (size_t)a.ldx * 4;  // float4s per 16-k block

  floatx4 acc = floatx4{0.f, 0.f, 0.f, 0.f};
  float4 af[3][UQ], bf[3][UQ];
#define BOA_DEC_LOAD(BUF, Q0)                                      \
  _Pragma("unroll") for (int q = 0; q < UQ; ++q) {                 \
    af[BUF][q] = wp[(size_t)((Q0) + q) * wq];                      \
    bf[BUF][q] = xp[(size_t)((Q0) + q) * xq];                      \
  }                                                                \
  __builtin_amdgcn_sched_barrier(0);
  BOA_DEC_LOAD(0, 0)
  if (G > 1) { BOA_DEC_LOAD(1, UQ) }
#pragma unroll
  for (int gi = 0; gi < G; ++gi) {
    if (gi + 2 < G) { BOA_DEC_LOAD((gi + 2) % 3, (gi + 2) * UQ) }
#pragma unroll
    for (int q = 0; q < UQ; ++q) {
      const float4 av = af[gi % 3][q], bv = bf[gi % 3][q];
      acc = __builtin_amdgcn_mfma_f32_16x16x4f32(av.x, bv.x, acc, 0, 0, 0);
      acc = __builtin_amdgcn_mfma_f32_16x16x4f32(av.y, bv.y, acc, 0, 0, 0);
      acc = __builtin_amdgcn_mfma_f32_16x16x4f32(av.z, bv.z, acc, 0, 0, 0);
      acc = __builtin_amdgcn_mfma_f32_16x16x4f32(av.w, bv.w, acc, 0, 0, 0);
    }
    __builtin_amdgcn_sched_barrier(0);
  }
#undef BOA_DEC_LOAD

  // Epilogue: acc + bias, activation, + residual.  CONV mode runs the causal
  // conv step on the x half of in_proj and stores the z half.
  const int m = m0 + i;
  if (m >= a.M) return;
  int nf[4];
#pragma unroll
  for (int e = 0; e < 4; ++e) nf[e] = a.row_major ? n0 + 4 * g + e : n0 + 4 * e + g;
  float v[4];
#pragma unroll
  for (int e = 0; e < 4; ++e) {
    const int n = min(nf[e], a.N - 1);
    float r = acc[e] + (a.bias ? a.bias[n] : 0.0f);
    if (a.act == ACT_GELU) r = gelu(r);
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
  const bool full = n0 + 16 <= a.N;
  if (a.conv_di > 0 && n0 < a.conv_di) {
    float cv[4];
#pragma unroll
    for (int e = 0; e < 4; ++e) {
      const int n = nf[e];
      float4* st = reinterpret_cast<float4*>(a.conv_state) + (size_t)n * a.ld_state + m;
      const float4 s0 = *st;
      const float4 wv = reinterpret_cast<const float4*>(a.conv_w)[n];
      cv[e] = conv_step_value(a.conv_b[n], s0, v[e], wv);
      *st = make_float4(s0.y, s0.z, s0.w, v[e]);
    }
    float* o = a.conv_out + ((size_t)(n0 >> 4) * a.ldc + m) * 16 + 4 * g;
    *reinterpret_cast<float4*>(o) = make_float4(cv[0], cv[1], cv[2], cv[3]);
    return;
  }
  const int row0 = a.conv_di > 0 ? n0 - a.conv_di : n0;
  float* o = a.C + ((size_t)(row0 >> 4) * a.ldc + m) * 16 + 4 * g;
  if (a.res) {
    const float4 rv =
        *reinterpret_cast<const float4*>(a.res + ((size_t)(n0 >> 4) * a.ldr + m) * 16 + 4 * g);
    v[0] = v[0] + rv.x; v[1] = v[1] + rv.y; v[2] = v[2] + rv.z; v[3] = v[3] + rv.w;
  }
  if (full) {
    *reinterpret_cast<float4*>(o) = make_float4(v[0], v[1], v[2], v[3]);
  } else {
#pragma unroll
    for (int e = 0; e < 4; ++e)
      if (nf[e] < a.N) o[e] = v[e];
  }
}

hipError_t dec_gemm(const DecGemmArgs& a, hipStream_t s) {
  if (a.M <= 0 || a.N <= 0) return hipSuccess;
  if (a.ldw < (a.N + 15) / 16 * 16 || a.ldx < a.M || a.ldc < (a.row_major ? a.N : a.M) ||
      (a.res && a.ldr < a.M) || (a.conv_di % 16))
    return hipErrorInvalidValue;
  const int tiles = ((a.N + 15) / 16) * ((a.M + 15) / 16);
  const dim3 grid((tiles + 3) / 4), block(256);
  switch (a.K) {
    case 64: hipLaunchKernelGGL((dec_gemm_kernel<16>), grid, block, 0, s, a); break;
    case 128: hipLaunchKernelGGL((dec_gemm_kernel<32>), grid, block, 0, s, a); break;
    case 256: hipLaunchKernelGGL((dec_gemm_kernel<64>), grid, block, 0, s, a); break;
    case 512: hipLaunchKernelGGL((dec_gemm_kernel<128>), grid, block, 0, s, a); break;
    case 1024: hipLaunchKernelGGL((dec_gemm_kernel<256>), grid, block, 0, s, a); break;
    case 2048: hipLaunchKernelGGL((dec_gemm_kernel<512>), grid, block, 0, s, a); break;
    default: return hipErrorInvalidValue;  // decode needs d_model a power of two >= 16
  }
  return hipGetLastError();
}

// Weight relayout for decode: W [K][ldw_in] row-major (the compress layout)
// -> k-blocked [K/16][ldn][16]; with `permute`, tile row j of every 16-row
// output tile holds feature (j & ~15) + dperm(j & 15) (dperm is its own
// inverse).
__global__ void dec_weight_blk_kernel(const float* __restrict__ w, int ldw_in, float* out, int K,
                                      int ldn, int permute) {
  const size_t idx = (size_t)blockIdx.x * blockDim.x + threadIdx.x;
  if (idx >= (size_t)K * ldn) return;
  const int k = (int)(idx / ldn), j = (int)(idx % ldn);
  const int n = permute ? (j & ~15) + dperm(j & 15) : j;
  out[dblk(k, j, ldn)] = w[(size_t)k * ldw_in + n];
}

hipError_t launch_dec_weight_blk(const float* w, int ldw_in, float* out, int K, int ldn,
                                 int permute, hipStream_t s) {
  if (K % 16 || ldn % 16 || ldn > ldw_in) return hipErrorInvalidValue;
  const size_t n = (size_t)K * ldn;
  hipLaunchKernelGGL(dec_weight_blk_kernel, dim3((unsigned)((n + 255) / 256)), dim3(256), 0, s, w,
                     ldw_in, out, K, ldn, permute);
  return hipGetLastError();
}

// -------------------------------------------------------------- LayerNorm
// A 256-thread block normalises DEC_LN_MB lanes: the [d][MB] slab of the
// features-major input is staged in LDS with coalesced row segments (row
// stride MB+1), the statistics are computed in the reference's order, and
// the normalised slab is written back coalesced.
//   LN1 (mode 1): one 32-lane half-wave per lane; lane l sums elements l,
//     l+32, ... in order, then the shuffle-down tree 16..1 (the
//     reference's warp-per-row order, as in the compress LN1 kernel).
//   LN2 (mode 2): one thread per lane sums all elements in order.
// Layer 0's LN1 also gathers the embedding rows (and stores x^T).
constexpr int DEC_LN_MB = 16;
constexpr int DEC_LN_S = DEC_LN_MB + 1;

template <int MODE>
__global__ __launch_bounds__(256) void dec_ln_kernel(const float* __restrict__ emb,
                                                     const uint8_t* __restrict__ tok, float* xt,
                                                     const float* src, float* xnt,
                                                     const float* __restrict__ w,
                                                     const float* __restrict__ b, int M, int d,
                                                     int ld, int* t_counter) {
  __shared__ float tile[512 * DEC_LN_S];
  __shared__ float stats[2 * DEC_LN_MB];
  if (t_counter && blockIdx.x == 0 && threadIdx.x == 0) *t_counter += 1;
  const int m0 = blockIdx.x * DEC_LN_MB;
  const int nm = min(DEC_LN_MB, M - m0);
  for (int q = threadIdx.x; q < d * DEC_LN_MB; q += blockDim.x) {
    // q -> (feature block, lane, feature in block): contiguous in memory
    const int i = (q / (16 * DEC_LN_MB)) * 16 + (q % 16), j = (q / 16) % DEC_LN_MB;
    float v = 0.0f;
    if (j < nm) {
      const int m = m0 + j;
      if (emb) {
        v = emb[(size_t)tok[m] * d + i];
        xt[dblk(i, m, ld)] = v;
      } else {
        v = src[dblk(i, m, ld)];
      }
    }
    tile[i * DEC_LN_S + j] = v;
  }
  __syncthreads();
  if (MODE == 1) {
    const int half = threadIdx.x >> 5, l = threadIdx.x & 31;
    for (int j = half; j < DEC_LN_MB; j += 8) {
      float sum = 0.0f, sq = 0.0f;
      for (int idx = l; idx < d; idx += 32) {
        const float v = tile[idx * DEC_LN_S + j];
        sum = sum + v;
        sq = sq + v * v;
      }
#pragma unroll
      for (int off = 16; off > 0; off >>= 1) {
        sum = sum + __shfl_down(sum, off, 32);
        sq = sq + __shfl_down(sq, off, 32);
      }
      if (l == 0) {
        const float mean = sum / (float)d;
        const float var = sq / (float)d - mean * mean;
        stats[2 * j] = mean;
        stats[2 * j + 1] = 1.0f / __builtin_sqrtf(var + 1e-5f);
      }
    }
  } else if (threadIdx.x < DEC_LN_MB) {
    const int j = threadIdx.x;
    float sum = 0.0f, sq = 0.0f;
    for (int idx = 0; idx < d; ++idx) {
      const float v = tile[idx * DEC_LN_S + j];
      sum = sum + v;
      sq = sq + v * v;
    }
    const float mean = sum / (float)d;
    const float var = sq / (float)d - mean * mean;
    stats[2 * j] = mean;
    stats[2 * j + 1] = 1.0f / __builtin_sqrtf(var + 1e-5f);
  }
  __syncthreads();
  for (int q = threadIdx.x; q < d * DEC_LN_MB; q += blockDim.x) {
    const int i = (q / (16 * DEC_LN_MB)) * 16 + (q % 16), j = (q / 16) % DEC_LN_MB;
    if (j < nm) {
      const float v = tile[i * DEC_LN_S + j];
      xnt[dblk(i, m0 + j, ld)] = ((v - stats[2 * j]) * stats[2 * j + 1]) * w[i] + b[i];
    }
  }
}

hipError_t launch_dec_ln1(const float* emb, const uint8_t* tok, float* xt, float* xnt,
                          const float* w, const float* b, int M, int d, int ld, int* t_counter,
                          hipStream_t s) {
  if (d > 512) return hipErrorInvalidValue;
  hipLaunchKernelGGL(dec_ln_kernel<1>, dim3((M + DEC_LN_MB - 1) / DEC_LN_MB), dim3(256), 0, s, emb,
                     tok, xt, xt, xnt, w, b, M, d, ld, t_counter);
  return hipGetLastError();
}

hipError_t launch_dec_ln2(const float* xt, float* xnt, const float* w, const float* b, int M, int d,
                          int ld, hipStream_t s) {
  if (d > 512) return hipErrorInvalidValue;
  hipLaunchKernelGGL(dec_ln_kernel<2>, dim3((M + DEC_LN_MB - 1) / DEC_LN_MB), dim3(256), 0, s,
                     nullptr, nullptr, nullptr, xt, xnt, w, b, M, d, ld, nullptr);
  return hipGetLastError();
}

// ------------------------------------------------------------------- scan
// Thread t of block (x, y): channel c = 16 y + t % 16, lane m = 16 x + t / 16
// (16 lanes per block); the k-blocked state keeps h[c][n][m] at
// ((c/16 * ds + n) * ld_state + m) * 16 + c % 16.
template <int DS, int RB>
__global__ __launch_bounds__(256) void dec_scan_kernel(LayerW Lw, const float* __restrict__ zt,
                                                       const float* __restrict__ cvt,
                                                       const float* __restrict__ deltat,
                                                       float* ssm, float* yt, int M, int ld,
                                                       int ld_state, int r, int di) {
  const int cl = threadIdx.x & 15;
  const int c = blockIdx.y * 16 + cl;
  const int m = blockIdx.x * 16 + (threadIdx.x >> 4);
  if (m >= M) return;
  ScanCtx<DS, RB> sc;
#pragma unroll
  for (int j = 0; j < RB; ++j) sc.wdt[j] = j < r ? Lw.w_dt[(size_t)j * di + c] : 0.0f;
  float* h = ssm + ((size_t)blockIdx.y * DS * ld_state + m) * 16 + cl;
#pragma unroll
  for (int n = 0; n < DS; ++n) {
    sc.na[n] = Lw.neg_exp_a[(size_t)c * DS + n];
    sc.h[n] = h[(size_t)n * ld_state * 16];
  }
  sc.bdt = Lw.b_dt[c];
  sc.dd = Lw.dd[c];
  float drow[RB + 2 * DS];
#pragma unroll
  for (int j = 0; j < RB; ++j) drow[j] = j < r ? deltat[dblk(j, m, ld)] : 0.0f;
#pragma unroll
  for (int j = 0; j < 2 * DS; ++j) drow[RB + j] = deltat[dblk(r + j, m, ld)];
  const float u = cvt[dblk(c, m, ld)];
  const float z = zt[dblk(c, m, ld)];
  yt[dblk(c, m, ld)] = scan_token<DS, RB>(sc, drow, drow + RB, r, u, z);
#pragma unroll
  for (int n = 0; n < DS; ++n) h[(size_t)n * ld_state * 16] = sc.h[n];
}

hipError_t launch_dec_scan(const Dims& D, const LayerW& Lw, const float* zt, const float* cvt,
                           const float* deltat, float* ssm, float* yt, int M, int ld, int ld_state,
                           hipStream_t s) {
  if (D.di % 16) return hipErrorInvalidValue;
  dim3 grid((M + 15) / 16, D.di / 16);
#define BOA_DEC_SCAN(DSv, RBv)                                                                \
  hipLaunchKernelGGL((dec_scan_kernel<DSv, RBv>), grid, dim3(256), 0, s, Lw, zt, cvt, deltat, \
                     ssm, yt, M, ld, ld_state, D.r, D.di)
  if (D.ds == 16) {
    if (D.r <= 8) BOA_DEC_SCAN(16, 8);
    else if (D.r <= 16) BOA_DEC_SCAN(16, 16);
    else BOA_DEC_SCAN(16, 32);
  } else if (D.ds == 32) {
    if (D.r <= 8) BOA_DEC_SCAN(32, 8);
    else if (D.r <= 16) BOA_DEC_SCAN(32, 16);
    else BOA_DEC_SCAN(32, 32);
  } else {
    return hipErrorInvalidValue;
  }
#undef BOA_DEC_SCAN
  return hipGetLastError();
}

// --------------------------------------------------- state layout changes
// chunk layout: conv [lane][c][4], ssm [lane][c][n]
// step layout:  conv [c][lane][4], ssm [c/16][n][lane][c%16] (lane stride ld_state)
__global__ void state_to_step_kernel(const float* conv_in, const float* ssm_in, float* conv_out,
                                     float* ssm_out, int lanes, int di, int ds, int ld_state) {
  const int idx = blockIdx.x * blockDim.x + threadIdx.x;
  if (idx >= lanes * di) return;
  const int b = idx / di, c = idx % di;
  reinterpret_cast<float4*>(conv_out)[(size_t)c * ld_state + b] =
      reinterpret_cast<const float4*>(conv_in)[idx];
  for (int n = 0; n < ds; ++n)
    ssm_out[(((size_t)(c >> 4) * ds + n) * ld_state + b) * 16 + (c & 15)] =
        ssm_in[(size_t)idx * ds + n];
}

__global__ void state_to_chunk_kernel(const float* conv_in, const float* ssm_in, float* conv_out,
                                      float* ssm_out, int lanes, int di, int ds, int ld_state) {
  const int idx = blockIdx.x * blockDim.x + threadIdx.x;
  if (idx >= lanes * di) return;
  const int b = idx / di, c = idx % di;
  reinterpret_cast<float4*>(conv_out)[idx] =
      reinterpret_cast<const float4*>(conv_in)[(size_t)c * ld_state + b];
  for (int n = 0; n < ds; ++n)
    ssm_out[(size_t)idx * ds + n] =
        ssm_in[(((size_t)(c >> 4) * ds + n) * ld_state + b) * 16 + (c & 15)];
}

hipError_t launch_state_relayout(const float* conv_in, const float* ssm_in, float* conv_out,
                                 float* ssm_out, int lanes, int di, int ds, int ld_state,
                                 bool to_step, hipStream_t s) {
  const int n = lanes * di;
  if (to_step)
    hipLaunchKernelGGL(state_to_step_kernel, dim3((n + 255) / 256), dim3(256), 0, s, conv_in,
                       ssm_in, conv_out, ssm_out, lanes, di, ds, ld_state);
  else
    hipLaunchKernelGGL(state_to_chunk_kernel, dim3((n + 255) / 256), dim3(256), 0, s, conv_in,
                       ssm_in, conv_out, ssm_out, lanes, di, ds, ld_state);
  return hipGetLastError();
}

}  // namespace boa
