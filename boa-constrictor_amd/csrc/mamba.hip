// Mamba-v1 block kernels: LayerNorms, causal depthwise conv1d + SiLU, and the
// fused dt_proj + softplus + selective scan + D + SiLU(z) gate, each in a
// chunk (teacher-forced tile, sequential in t) and a step (one token per
// lane) form that share one per-element operation sequence.
//
// Reference semantics followed (portability_solved_cpp/):
//   LN1  inference_kernels.cu:293-348  32-lane shuffle-down tree sums
//   LN2  inference_kernels.cu:229-277  sequential per-row sums
//   conv mamba_kernels.cu:158-197 (step), 370-412 (chunk)
//   scan mamba_kernels.cu:271-352 (step), 414-470 (chunk), with the dt_proj
//        GEMM (K = dt_rank fma chain) + softplus of boa_gpu.hpp:317-318 and
//        the gate of mamba_kernels.cu:130-144
// rsqrtf is replaced by 1/sqrt with IEEE-rounded division and square root.
#include <algorithm>

#include "block_device.h"
#include "boa_kernels.h"

namespace boa {

// four consecutive activations (fp32 or bf16 storage)
__device__ __forceinline__ void ld4(const float* p, float* v) {
  const float4 t = *reinterpret_cast<const float4*>(p);
  v[0] = t.x; v[1] = t.y; v[2] = t.z; v[3] = t.w;
}
__device__ __forceinline__ void ld4(const uint16_t* p, float* v) {
  const ushort4 t = *reinterpret_cast<const ushort4*>(p);
  v[0] = bf16_to_f32(t.x); v[1] = bf16_to_f32(t.y); v[2] = bf16_to_f32(t.z); v[3] = bf16_to_f32(t.w);
}
__device__ __forceinline__ void st4(float* p, const float* v) {
  *reinterpret_cast<float4*>(p) = make_float4(v[0], v[1], v[2], v[3]);
}
__device__ __forceinline__ void st4(uint16_t* p, const float* v) {
  *reinterpret_cast<ushort4*>(p) =
      make_ushort4(f32_to_bf16(v[0]), f32_to_bf16(v[1]), f32_to_bf16(v[2]), f32_to_bf16(v[3]));
}

// -------------------------------------------------------------- LayerNorm
// Both kernels stage a block of rows in LDS with 16-byte loads (every load of
// a thread issued before the first is used), take the statistics in the
// reference's order from LDS, and store 16-byte (fp32) or 8-byte (bf16)
// groups of the normalised rows.

// LN1: 8 rows per 256-thread block; half-wave h sums row h as the
// reference's warp-per-row reduction does: lane l accumulates elements l,
// l+32, ... (those below D) in order, then the shuffle-down tree 16, 8, 4,
// 2, 1, lane 0's
// totals broadcast.  Layer 0 gathers the embedding rows of the tile's
// tokens and also stores them as x.
// Rows are D wide, of which the model's n <= D features are real: a model
// of d_model n is run at the next width D the kernels are built for, its
// features n .. D-1 zero (weights and activations).  Those zeros add +0 to
// the sums, which leaves them unchanged, and the mean and variance divide
// by n, so the statistics are the n-feature row's.
template <typename TO, int D>
__global__ __launch_bounds__(256) void ln1_kernel(const float* __restrict__ emb, TokenSrc tok,
                                                  int use_tok, int T, int t0, float* x, TO* xn,
                                                  const float* __restrict__ w,
                                                  const float* __restrict__ b, int rows, int n) {
  constexpr int RPB = 8, S = D + 4, DQ = D / 4;
  constexpr int NQ = (RPB * DQ + 255) / 256;
  __shared__ __align__(16) float tile[RPB * S];
  const int r0 = blockIdx.x * RPB, tid = threadIdx.x;
  float4 buf[NQ];
#pragma unroll
  for (int i = 0; i < NQ; ++i) {
    const int q = tid + 256 * i, r = q / DQ, c4 = q % DQ;
    if (q < RPB * DQ && r0 + r < rows) {
      const float* src = x + (size_t)(r0 + r) * D;
      if (use_tok) {
        const int row = r0 + r, lane = row / T, t = row % T;
        const int64_t pos = (int64_t)lane * tok.stride + t0 + t;
        const uint32_t token = (t0 + t < tok.len && pos < tok.total) ? tok.base[pos] : 0u;
        src = emb + (size_t)token * D;
      }
      buf[i] = *reinterpret_cast<const float4*>(src + 4 * c4);
    }
  }
#pragma unroll
  for (int i = 0; i < NQ; ++i) {
    const int q = tid + 256 * i, r = q / DQ, c4 = q % DQ;
    if (q < RPB * DQ && r0 + r < rows) {
      *reinterpret_cast<float4*>(tile + r * S + 4 * c4) = buf[i];
      if (use_tok) *reinterpret_cast<float4*>(x + (size_t)(r0 + r) * D + 4 * c4) = buf[i];
    }
  }
  __syncthreads();
  const int h = tid >> 5, l = tid & 31;
  float* row = tile + h * S;
  float sum = 0.0f, sq = 0.0f;
#pragma unroll
  for (int e = 0; e < (D + 31) / 32; ++e) {
    const int idx = l + 32 * e;
    if (D % 32 == 0 || idx < D) {
      const float v = row[idx];
      sum = sum + v;
      sq = sq + v * v;
    }
  }
#pragma unroll
  for (int off = 16; off > 0; off >>= 1) {
    sum = sum + __shfl_down(sum, off, 32);
    sq = sq + __shfl_down(sq, off, 32);
  }
  sum = __shfl(sum, 0, 32);
  sq = __shfl(sq, 0, 32);
  const float mean = sum / (float)n;
  const float var = sq / (float)n - mean * mean;
  const float inv_std = 1.0f / __builtin_sqrtf(var + 1e-5f);
#pragma unroll
  for (int e = 0; e < (D + 31) / 32; ++e) {
    const int idx = l + 32 * e;
    if (D % 32 == 0 || idx < D) row[idx] = ((row[idx] - mean) * inv_std) * w[idx] + b[idx];
  }
  __syncthreads();
#pragma unroll
  for (int i = 0; i < NQ; ++i) {
    const int q = tid + 256 * i, r = q / DQ, c4 = q % DQ;
    if (q < RPB * DQ && r0 + r < rows) st4(xn + (size_t)(r0 + r) * D + 4 * c4, tile + r * S + 4 * c4);
  }
}

// LN1 with the row in registers (D a multiple of 32): half-wave h of a
// block owns row 8 blockIdx + h and lane l holds elements l, l + 32, ...,
// read and written as one 32-element access per step; the sums, the
// shuffle tree and the normalisation are ln1_kernel's, without its LDS
// round trip and barriers.
template <typename TO, int D>
__global__ __launch_bounds__(256) void ln1_reg_kernel(const float* __restrict__ emb, TokenSrc tok,
                                                      int use_tok, int T, int t0, float* x, TO* xn,
                                                      const float* __restrict__ w,
                                                      const float* __restrict__ b, int rows, int n) {
  constexpr int E = D / 32;
  static_assert(D % 32 == 0, "whole 32-element steps");
  const int h = threadIdx.x >> 5, l = threadIdx.x & 31;
  const int r = blockIdx.x * 8 + h;
  if (r >= rows) return;  // no barriers below
  const float* src = x + (size_t)r * D;
  if (use_tok) {
    const int lane = r / T, t = r % T;
    const int64_t pos = (int64_t)lane * tok.stride + t0 + t;
    const uint32_t token = (t0 + t < tok.len && pos < tok.total) ? tok.base[pos] : 0u;
    src = emb + (size_t)token * D;
  }
  float v[E];
#pragma unroll
  for (int e = 0; e < E; ++e) v[e] = src[l + 32 * e];
  if (use_tok) {
#pragma unroll
    for (int e = 0; e < E; ++e) x[(size_t)r * D + l + 32 * e] = v[e];
  }
  float sum = 0.0f, sq = 0.0f;
#pragma unroll
  for (int e = 0; e < E; ++e) {
    sum = sum + v[e];
    sq = sq + v[e] * v[e];
  }
#pragma unroll
  for (int off = 16; off > 0; off >>= 1) {
    sum = sum + __shfl_down(sum, off, 32);
    sq = sq + __shfl_down(sq, off, 32);
  }
  sum = __shfl(sum, 0, 32);
  sq = __shfl(sq, 0, 32);
  const float mean = sum / (float)n;
  const float var = sq / (float)n - mean * mean;
  const float inv_std = 1.0f / __builtin_sqrtf(var + 1e-5f);
#pragma unroll
  for (int e = 0; e < E; ++e) {
    const int idx = l + 32 * e;
    const float o = ((v[e] - mean) * inv_std) * w[idx] + b[idx];
    if constexpr (sizeof(TO) == 2) xn[(size_t)r * D + idx] = f32_to_bf16(o);
    else xn[(size_t)r * D + idx] = o;
  }
}

hipError_t launch_ln1(const float* emb, TokenSrc tok, int T, int t0, float* x, void* xn,
                      const float* w, const float* b, int rows, int d, int n, bool bf16,
                      hipStream_t s) {
  const dim3 grid((rows + 7) / 8), block(256);
  const int ut = emb ? 1 : 0;
  // widths that are multiples of 32: the row in registers (C5 probe at
  // 8192 lanes: LN1 52 -> 27 ms per compress, 3.71 -> 3.80 MB/s; same bits)
#define BOA_LN1R(Dv)                                                                         \
  if (bf16)                                                                                  \
    BOA_LAUNCH((ln1_reg_kernel<uint16_t, Dv>), grid, block, 0, s, emb, tok, ut, T, t0, x,    \
               (uint16_t*)xn, w, b, rows, n);                                                \
  else                                                                                       \
    BOA_LAUNCH((ln1_reg_kernel<float, Dv>), grid, block, 0, s, emb, tok, ut, T, t0, x,       \
               (float*)xn, w, b, rows, n);                                                   \
  return hipGetLastError();
  switch (d) {
    case 64: BOA_LN1R(64)
    case 128: BOA_LN1R(128)
    case 256: BOA_LN1R(256)
    case 512: BOA_LN1R(512)
    case 80:  // the row through LDS
      if (bf16)
        BOA_LAUNCH((ln1_kernel<uint16_t, 80>), grid, block, 0, s, emb, tok, ut, T, t0, x,
                   (uint16_t*)xn, w, b, rows, n);
      else
        BOA_LAUNCH((ln1_kernel<float, 80>), grid, block, 0, s, emb, tok, ut, T, t0, x,
                   (float*)xn, w, b, rows, n);
      return hipGetLastError();
    default: return hipErrorInvalidValue;
  }
#undef BOA_LN1R
}

// LN2: per-row sums in element order (the reference's thread-per-row order).
// RPB rows per 256-thread block; thread t < RPB runs row t's sequential
// sums over the LDS copy (row stride D + 1 keeps those reads conflict-free).
// In place is allowed.  n <= D real features, as ln1_kernel.
template <typename T, int D>
__global__ __launch_bounds__(256) void ln2_kernel(const T* x, T* out, const float* __restrict__ w,
                                                  const float* __restrict__ b, int rows, int n) {
  constexpr int RPB = D <= 256 ? 32 : 16, S = D + 1, DQ = D / 4;
  constexpr int NQ = (RPB * DQ + 255) / 256;
  __shared__ float tile[RPB * S];
  __shared__ float stats[2 * RPB];
  const int r0 = blockIdx.x * RPB, tid = threadIdx.x;
  float v[NQ][4];
#pragma unroll
  for (int i = 0; i < NQ; ++i) {
    const int q = tid + 256 * i, r = q / DQ, c4 = q % DQ;
    if (q < RPB * DQ && r0 + r < rows) ld4(x + (size_t)(r0 + r) * D + 4 * c4, v[i]);
  }
#pragma unroll
  for (int i = 0; i < NQ; ++i) {
    const int q = tid + 256 * i, r = q / DQ, c4 = q % DQ;
    if (q < RPB * DQ && r0 + r < rows) {
      float* dst = tile + r * S + 4 * c4;
      dst[0] = v[i][0]; dst[1] = v[i][1]; dst[2] = v[i][2]; dst[3] = v[i][3];
    }
  }
  __syncthreads();
  if (tid < RPB && r0 + tid < rows) {
    const float* row = tile + tid * S;
    float s = 0.0f, q = 0.0f;
    for (int i = 0; i < D; ++i) {
      const float e = row[i];
      s = s + e;
      q = q + e * e;
    }
    const float mean = s / (float)n;
    const float var = q / (float)n - mean * mean;
    stats[2 * tid] = mean;
    stats[2 * tid + 1] = 1.0f / __builtin_sqrtf(var + 1e-5f);
  }
  __syncthreads();
#pragma unroll
  for (int i = 0; i < NQ; ++i) {
    const int q = tid + 256 * i, r = q / DQ, c4 = q % DQ;
    if (q < RPB * DQ && r0 + r < rows) {
      const float mean = stats[2 * r], inv_std = stats[2 * r + 1];
      const float* src = tile + r * S + 4 * c4;
      const float4 wv = *reinterpret_cast<const float4*>(w + 4 * c4);
      const float4 bv = *reinterpret_cast<const float4*>(b + 4 * c4);
      float o[4];
      o[0] = ((src[0] - mean) * inv_std) * wv.x + bv.x;
      o[1] = ((src[1] - mean) * inv_std) * wv.y + bv.y;
      o[2] = ((src[2] - mean) * inv_std) * wv.z + bv.z;
      o[3] = ((src[3] - mean) * inv_std) * wv.w + bv.w;
      st4(out + (size_t)(r0 + r) * D + 4 * c4, o);
    }
  }
}

// LN2 of bf16 rows, 64 rows per 256-thread block: the rows stay bf16 in
// LDS (D / 2 + 1 words a row, an odd stride, so that lane r's serial reads
// of row r fall on distinct banks), lane r of wave 0 runs row r's sums in
// element order as ln2_kernel's thread r does (a bf16 value converts to
// float exactly, so the sums and statistics are ln2_kernel's), then every
// thread normalises 16-byte groups.  Four times the rows per serial pass
// and twice the rows per CU of ln2_kernel's 16-row blocks.
template <int D>
__global__ __launch_bounds__(256) void ln2_b16_rows_kernel(const uint16_t* x, uint16_t* out,
                                                           const float* __restrict__ w,
                                                           const float* __restrict__ b, int rows,
                                                           int n) {
  constexpr int RPB = 64, SW = D / 2 + 1, DC = D / 8;  // words a row, 16-byte groups a row
  constexpr int NQ = RPB * DC / 256;
  static_assert(RPB * DC % 256 == 0, "whole groups per thread");
  __shared__ uint32_t tile[RPB * SW];
  __shared__ float stats[2 * RPB];
  const int r0 = blockIdx.x * RPB, tid = threadIdx.x;
  lds_u32x4 v[NQ];
#pragma unroll
  for (int i = 0; i < NQ; ++i) {
    const int q = tid + 256 * i, r = q / DC, c = q % DC;
    if (r0 + r < rows) v[i] = *reinterpret_cast<const lds_u32x4*>(x + (size_t)(r0 + r) * D + 8 * c);
  }
#pragma unroll
  for (int i = 0; i < NQ; ++i) {
    const int q = tid + 256 * i, r = q / DC, c = q % DC;
    if (r0 + r < rows) {
      uint32_t* dst = tile + r * SW + 4 * c;
      dst[0] = v[i][0]; dst[1] = v[i][1]; dst[2] = v[i][2]; dst[3] = v[i][3];
    }
  }
  __syncthreads();
  if (tid < RPB && r0 + tid < rows) {
    const uint32_t* row = tile + tid * SW;
    float s = 0.0f, q = 0.0f;
    for (int j = 0; j < D / 2; ++j) {
      const uint32_t wv = row[j];
      const float e0 = u2f(wv << 16), e1 = u2f(wv & 0xFFFF0000u);  // elements 2 j, 2 j + 1
      s = s + e0;
      q = q + e0 * e0;
      s = s + e1;
      q = q + e1 * e1;
    }
    const float mean = s / (float)n;
    const float var = q / (float)n - mean * mean;
    stats[2 * tid] = mean;
    stats[2 * tid + 1] = 1.0f / __builtin_sqrtf(var + 1e-5f);
  }
  __syncthreads();
#pragma unroll
  for (int i = 0; i < NQ; ++i) {
    const int q = tid + 256 * i, r = q / DC, c = q % DC;
    if (r0 + r < rows) {
      const float mean = stats[2 * r], inv_std = stats[2 * r + 1];
      const uint32_t* src = tile + r * SW + 4 * c;
      float o[8];
#pragma unroll
      for (int k = 0; k < 4; ++k) {
        const uint32_t wv = src[k];
        o[2 * k] = u2f(wv << 16);
        o[2 * k + 1] = u2f(wv & 0xFFFF0000u);
      }
#pragma unroll
      for (int e = 0; e < 8; ++e) o[e] = ((o[e] - mean) * inv_std) * w[8 * c + e] + b[8 * c + e];
      uint16_t* dst = out + (size_t)(r0 + r) * D + 8 * c;
      st4(dst, o);
      st4(dst + 4, o + 4);
    }
  }
}

hipError_t launch_ln2(const void* x, void* out, const float* w, const float* b, int rows, int d,
                      int n, bool bf16, hipStream_t s) {
#define BOA_LN2(Dv)                                                                             \
  {                                                                                             \
    constexpr int RPB = Dv <= 256 ? 32 : 16;                                                    \
    const dim3 grid((rows + RPB - 1) / RPB), block(256);                                        \
    if (bf16)                                                                                   \
      BOA_LAUNCH((ln2_kernel<uint16_t, Dv>), grid, block, 0, s, (const uint16_t*)x,     \
                         (uint16_t*)out, w, b, rows, n);                                        \
    else                                                                                        \
      BOA_LAUNCH((ln2_kernel<float, Dv>), grid, block, 0, s, (const float*)x,           \
                         (float*)out, w, b, rows, n);                                              \
  }
  // bf16 at width 512 (C5): 64-row blocks (C5 probe at 8192 lanes: LN2
  // 44 -> 21 ms per compress, compress 3.59 -> 3.66 MB/s; same bits)
  if (bf16 && d == 512) {
    BOA_LAUNCH((ln2_b16_rows_kernel<512>), dim3((rows + 63) / 64), dim3(256), 0, s,
               (const uint16_t*)x, (uint16_t*)out, w, b, rows, n);
    return hipGetLastError();
  }
  switch (d) {
    case 64: BOA_LN2(64) break;
    case 80: BOA_LN2(80) break;
    case 128: BOA_LN2(128) break;
    case 256: BOA_LN2(256) break;
    case 512: BOA_LN2(512) break;
    default: return hipErrorInvalidValue;
  }
#undef BOA_LN2
  return hipGetLastError();
}

// ------------------------------------------------------------------ conv1d
// The conv is no recurrence (an output needs its own input and the three
// before it), so a thread takes TB consecutive tokens of CP adjacent
// channels, reading the three inputs before its block from xz (or, for the
// first block, from the state).  The first block's thread also writes the
// new state, the last four inputs of (old state, tile), after having read
// the old one, so no other thread touches the state.  Against one thread per
// channel walking the whole tile: C2 probe 27.8 -> 26.4 ms per compress,
// C1 4.3 -> 0.47 ms.  A thread takes up to 128 tokens, in condition-free
// sub-blocks of eight loads in flight, as long as about a million threads
// remain (against eight tokens per thread: C3 probe 19.2 -> 16.4 ms, C5
// probe 155 -> 103 ms; C1, C2 the same), and CP adjacent channels: four in
// fp32 (16-byte accesses), two in bf16 (4-byte accesses).

// CP consecutive activations as floats (one 2 CP- or 4 CP-byte access)
template <int CP>
__device__ __forceinline__ void ldcp(const float* p, float* v) {
  if constexpr (CP == 1) {
    v[0] = *p;
  } else if constexpr (CP == 2) {
    const float2 t = *reinterpret_cast<const float2*>(p);
    v[0] = t.x; v[1] = t.y;
  } else {
    ld4(p, v);
  }
}
template <int CP>
__device__ __forceinline__ void ldcp(const uint16_t* p, float* v) {
  if constexpr (CP == 1) {
    v[0] = bf16_to_f32(*p);
  } else if constexpr (CP == 2) {
    const uint32_t t = *reinterpret_cast<const uint32_t*>(p);
    v[0] = u2f(t << 16); v[1] = u2f(t & 0xFFFF0000u);
  } else {
    ld4(p, v);
  }
}
template <int CP>
__device__ __forceinline__ void stcp(float* p, const float* v) {
  if constexpr (CP == 1) {
    *p = v[0];
  } else if constexpr (CP == 2) {
    *reinterpret_cast<float2*>(p) = make_float2(v[0], v[1]);
  } else {
    st4(p, v);
  }
}
template <int CP>
__device__ __forceinline__ void stcp(uint16_t* p, const float* v) {
  if constexpr (CP == 1) {
    *p = f32_to_bf16(v[0]);
  } else if constexpr (CP == 2) {
    *reinterpret_cast<uint32_t*>(p) =
        (uint32_t)f32_to_bf16(v[0]) | ((uint32_t)f32_to_bf16(v[1]) << 16);
  } else {
    st4(p, v);
  }
}

template <typename TA, int TB, int CP>
__global__ __launch_bounds__(256) void conv_chunk_tp_kernel(const TA* __restrict__ xz,
                                                            float* __restrict__ conv_state,
                                                            const float* __restrict__ w,
                                                            const float* __restrict__ cb,
                                                            TA* __restrict__ out, int lanes, int T,
                                                            int di, int ntb) {
  constexpr int SB = 8;  // tokens loaded together
  static_assert(TB % SB == 0, "whole sub-blocks");
  const int dq = di / CP;
  const int64_t idx = (int64_t)blockIdx.x * blockDim.x + threadIdx.x;
  if (idx >= (int64_t)lanes * ntb * dq) return;
  const int c = (int)(idx % dq) * CP;
  const int64_t rest = idx / dq;
  const int tb = (int)(rest % ntb), b = (int)(rest / ntb);
  const int t0 = tb * TB;
  constexpr int M = sizeof(TA) == 2 ? MATH_HW : MATH_BF;
  float4 wv[CP];
  float bias[CP];
#pragma unroll
  for (int k = 0; k < CP; ++k) {
    wv[k] = reinterpret_cast<const float4*>(w)[c + k];
    bias[k] = cb[c + k];
  }
  const TA* xp = xz + (size_t)b * T * (2 * di) + c;
  TA* op = out + (size_t)b * T * di + c;
  float4* st = reinterpret_cast<float4*>(conv_state) + (size_t)b * di + c;
  float4 s0[CP];
  float xm3[CP], xm2[CP], xm1[CP];
  if (tb == 0) {
#pragma unroll
    for (int k = 0; k < CP; ++k) {
      s0[k] = st[k];
      xm3[k] = s0[k].y; xm2[k] = s0[k].z; xm1[k] = s0[k].w;
    }
  } else {  // t0 >= TB >= 3
    ldcp<CP>(xp + (size_t)(t0 - 3) * 2 * di, xm3);
    ldcp<CP>(xp + (size_t)(t0 - 2) * 2 * di, xm2);
    ldcp<CP>(xp + (size_t)(t0 - 1) * 2 * di, xm1);
  }
  const int nt = min(TB, T - t0);
  int u = 0;
  // whole sub-blocks: SB loads in flight, no per-token conditions
#pragma unroll 1
  for (; u + SB <= nt; u += SB) {
    float xv[SB][CP];
#pragma unroll
    for (int v = 0; v < SB; ++v) ldcp<CP>(xp + (size_t)(t0 + u + v) * 2 * di, xv[v]);
#pragma unroll
    for (int v = 0; v < SB; ++v) {
      float o[CP];
#pragma unroll
      for (int k = 0; k < CP; ++k) {
        o[k] = conv_value<M>(bias[k], xm3[k], xm2[k], xm1[k], xv[v][k], wv[k]);
        xm3[k] = xm2[k]; xm2[k] = xm1[k]; xm1[k] = xv[v][k];
      }
      stcp<CP>(op + (size_t)(t0 + u + v) * di, o);
    }
  }
  for (; u < nt; ++u) {  // the tile's last tokens
    float x0[CP], o[CP];
    ldcp<CP>(xp + (size_t)(t0 + u) * 2 * di, x0);
#pragma unroll
    for (int k = 0; k < CP; ++k) {
      o[k] = conv_value<M>(bias[k], xm3[k], xm2[k], xm1[k], x0[k], wv[k]);
      xm3[k] = xm2[k]; xm2[k] = xm1[k]; xm1[k] = x0[k];
    }
    stcp<CP>(op + (size_t)(t0 + u) * di, o);
  }
  if (tb == 0) {
    // the last four of (s0.x, s0.y, s0.z, s0.w, x_0 .. x_{T-1})
    const int k0 = T < 4 ? T : 4;  // inputs of the tile among the last four
#pragma unroll
    for (int k = 0; k < CP; ++k) {
      float q[4] = {s0[k].x, s0[k].y, s0[k].z, s0[k].w};
      for (int i = 0; i < 4 - k0; ++i) q[i] = q[i + k0];
      for (int i = 0; i < k0; ++i) q[4 - k0 + i] = ldv(xp + (size_t)(T - k0 + i) * 2 * di + k);
      st[k] = make_float4(q[0], q[1], q[2], q[3]);
    }
  }
}

#ifndef BOA_CONV_CP_B16
#define BOA_CONV_CP_B16 2
#endif
#ifndef BOA_CONV_CP_F32
#define BOA_CONV_CP_F32 4
#endif
#ifndef BOA_CONV_MIN_THREADS
#define BOA_CONV_MIN_THREADS (1 << 20)
#endif

template <typename TA, int CP>
static hipError_t conv_go(const void* xz, float* conv_state, const float* w, const float* cb,
                          void* out, int lanes, int T, int di, hipStream_t s) {
  if (di % CP) return hipErrorInvalidValue;
  // tokens per thread: the most (up to 128) that still leave about a million
  // threads, which spreads a thread's weight loads and its three-input halo
  // over more outputs
  const int64_t per_tb = (int64_t)lanes * (di / CP);
  int TB = 128;
  while (TB > 8 && per_tb * ((T + TB - 1) / TB) < BOA_CONV_MIN_THREADS) TB /= 2;
  const int ntb = (T + TB - 1) / TB;
  const dim3 grid((unsigned)((per_tb * ntb + 255) / 256)), block(256);
  const TA* x = (const TA*)xz;
  TA* o = (TA*)out;
  switch (TB) {
    case 128: BOA_LAUNCH((conv_chunk_tp_kernel<TA, 128, CP>), grid, block, 0, s, x, conv_state, w, cb, o, lanes, T, di, ntb); break;
    case 64: BOA_LAUNCH((conv_chunk_tp_kernel<TA, 64, CP>), grid, block, 0, s, x, conv_state, w, cb, o, lanes, T, di, ntb); break;
    case 32: BOA_LAUNCH((conv_chunk_tp_kernel<TA, 32, CP>), grid, block, 0, s, x, conv_state, w, cb, o, lanes, T, di, ntb); break;
    case 16: BOA_LAUNCH((conv_chunk_tp_kernel<TA, 16, CP>), grid, block, 0, s, x, conv_state, w, cb, o, lanes, T, di, ntb); break;
    default: BOA_LAUNCH((conv_chunk_tp_kernel<TA, 8, CP>), grid, block, 0, s, x, conv_state, w, cb, o, lanes, T, di, ntb); break;
  }
  return hipGetLastError();
}

hipError_t launch_conv_chunk(const void* xz, float* conv_state, const float* w, const float* cb,
                             void* out, int lanes, int T, int di, bool bf16, hipStream_t s) {
  if (T <= 0) return hipSuccess;
  if (bf16) return conv_go<uint16_t, BOA_CONV_CP_B16>(xz, conv_state, w, cb, out, lanes, T, di, s);
  return conv_go<float, BOA_CONV_CP_F32>(xz, conv_state, w, cb, out, lanes, T, di, s);
}

// -------------------------------------------------------- selective scan
// Thread per (lane, channel); a block covers bs channels of one lane (bs
// divides di), so the token's delta row (dt_in | B | C) is the same for every
// thread of the wave and is read with scalar loads into SGPRs: no LDS
// staging and no barriers (against rows staged in LDS and read as
// broadcasts, 9 % faster in fp32 on the C2 model and 19-21 % in bf16 on the
// C3 and C5 models).  FULL: dt_rank equals the bound RB.  Otherwise the dt
// inputs beyond dt_rank are zeroed, which leaves the fma chain's value
// unchanged (the partial sum starts at +0 and so is never -0, and
// fma(0, 0, a) = a).  d_state 16 with dt_rank <= 16 runs five (fp32, 80
// VGPRs) or six (bf16) waves per SIMD.
template <int DS, int RB, bool FULL>
__device__ __forceinline__ void scan_row(const float* dr, int r, float* dv) {
#pragma unroll
  for (int j = 0; j < RB; ++j) {
    const float v = dr[j];  // j < RB <= R: inside the row
    dv[j] = FULL || j < r ? v : 0.0f;
  }
#pragma unroll
  for (int j = 0; j < 2 * DS; ++j) dv[RB + j] = dr[r + j];
}
// bf16 rows: dt_rank, d_state and so the row length are even (d_model is a
// multiple of 64), so the element pairs are read as aligned dwords
template <int DS, int RB, bool FULL>
__device__ __forceinline__ void scan_row(const uint16_t* dr, int r, float* dv) {
  const uint32_t* w = reinterpret_cast<const uint32_t*>(dr);
#pragma unroll
  for (int j = 0; j < RB / 2; ++j) {
    const uint32_t v = w[j];
    dv[2 * j] = FULL || 2 * j < r ? u2f(v << 16) : 0.0f;
    dv[2 * j + 1] = FULL || 2 * j + 1 < r ? u2f(v & 0xFFFF0000u) : 0.0f;
  }
  const uint32_t* wb = reinterpret_cast<const uint32_t*>(dr + r);
#pragma unroll
  for (int j = 0; j < DS; ++j) {
    const uint32_t v = wb[j];
    dv[RB + 2 * j] = u2f(v << 16);
    dv[RB + 2 * j + 1] = u2f(v & 0xFFFF0000u);
  }
}

template <int DS, int RB, bool FULL, typename TA>
__global__ __launch_bounds__(256) __attribute__((amdgpu_waves_per_eu(DS == 16 && RB <= 16 ? (sizeof(TA) == 2 ? 6 : 5) : 1, 8)))
void scan_chunk_sload_kernel(Dims D, LayerW Lw, const TA* __restrict__ xz,
                             const TA* __restrict__ conv, const TA* __restrict__ delta,
                             float* __restrict__ ssm_state, TA* __restrict__ y, int lanes,
                             int T) {
  const int di = D.di, R = D.R;
  const int base = blockIdx.x * blockDim.x;
  const int b = base / di;
  const int c = base - b * di + threadIdx.x;
  float* ssm = ssm_state + (size_t)(base + threadIdx.x) * DS;
  ScanCtx<DS, RB> sc;
  scan_load<DS, RB>(sc, Lw, ssm, c, di, D.r);
  const TA* drows = delta + (size_t)b * T * R;
  for (int t = 0; t < T; ++t) {
    const size_t row = (size_t)b * T + t;
    float dv[RB + 2 * DS];
    scan_row<DS, RB, FULL>(drows + (size_t)t * R, D.r, dv);
    const float u = ldv(conv + row * di + c);
    const float z = ldv(xz + row * 2 * di + di + c);
    stv(y + row * di + c, scan_token<DS, RB, sizeof(TA) == 2 ? MATH_HW : MATH_BF>(
                              sc, dv, dv + RB, RB, u, z));
  }
  scan_store<DS, RB>(sc, ssm);
}

// Token-blocked form for small grids (under one wave per SIMD with one
// thread per channel, e.g. d_model 64 with 64 lanes: 128 waves for 1024
// SIMDs, every token's latency exposed).  A block holds TBK_CPB channels of
// one lane, 16 threads each, and the work of a pass of TB tokens is split by
// kind instead of by state:
//   1. thread (c, k) computes tokens k, k + 16, ...'s scalars once: dt (the
//      dt_proj chain and softplus), D u and the gate z sigmoid(z);
//   2. thread (c, k) runs its SPT states through the pass's tokens,
//      h = (2^(na dt) h) + ((dt B) u), and leaves each token's h in LDS;
//   3. thread (c, k) sums y = y + h_n C_n over n = 0 .. DS-1 in order for
//      tokens k, k + 16, ..., adds D u, gates and stores.
// (bf16 at d_state 16: the fused update of scan_token,
// h = fma(2^(na dt), h, B (dt u)), y = fma(h_n, C_n, y).)
// Every element sees scan_token's operations in scan_token's order, so the
// bits are scan_chunk_sload_kernel's.  The per-token scalars are computed
// once per channel and the recurrence's critical path per token is its fma.
// The next pass's delta rows, u and z are loaded into registers while the
// current pass computes, so global latency is exposed once per kernel rather
// than per pass.  Within a wave the channel index runs fastest: u, z and y
// move as 64-byte rows, and the LDS strides below keep a wave's 64 lanes on
// distinct banks in phases 2 and 3.
// C1 (64 lanes, d_model 64): 4.7 ms of scan per compress, against 37.2 with
// one thread per channel and 28.6 with four threads per channel each owning
// four states (each recomputing the token's dt and gate, the output sum
// handed along by DPP).  On large grids the h round trip through LDS and the
// barriers cost more than they save: C2's 1000 lanes compress at 5.05 MB/s
// this way against 5.63 with one thread per channel, C3's 8192 bf16 lanes at
// 9.1 against 19.6; 250 lanes x 512 channels are even (4.89 both).
constexpr int TBK_CPB = 16;  // channels per block (di is a multiple of 16)

template <int DS>
struct TblkShape {
  static constexpr int G = 16, SPT = DS / G;
  static constexpr int TB = DS == 16 ? 32 : 16;  // tokens per pass
  static constexpr int TPT = TB / G;              // phase 1/3 tokens per thread
  static constexpr int HS = DS + 1;               // a token's h row
  // per-channel strides, 4 mod 64 words: lanes (c, k) of a wave land on
  // c * 4 + k (+ 17 k in phase 3) -- 64 distinct banks
  static constexpr int TSTR = TB * 4 + ((4 - TB * 4 % 64) + 64) % 64;
  static constexpr int CSTR = TB * HS + ((4 - TB * HS % 64) + 64) % 64;
  template <int RB>
  static constexpr int lds_floats() {
    return TB * (RB + 2 * DS) + TBK_CPB * TSTR + TBK_CPB * CSTR;
  }
};

template <int DS, int RB, typename TA>
__global__ __launch_bounds__(256) void scan_chunk_tblk_kernel(Dims D, LayerW Lw,
                                                              const TA* __restrict__ xz,
                                                              const TA* __restrict__ conv,
                                                              const TA* __restrict__ delta,
                                                              float* __restrict__ ssm_state,
                                                              TA* __restrict__ y, int lanes,
                                                              int T) {
  using S = TblkShape<DS>;
  constexpr int G = S::G, SPT = S::SPT, TB = S::TB, TPT = S::TPT, HS = S::HS;
  constexpr int NT = TBK_CPB * G;                   // threads
  constexpr int ND = (TB * (RB + 2 * DS) + NT - 1) / NT;  // delta staging loads per thread
  static_assert(DS % G == 0 && TB % G == 0, "whole states and tokens per thread");
  constexpr int M = sizeof(TA) == 2 ? MATH_HW : MATH_BF;
  extern __shared__ __align__(16) float smem[];  // s_tok is read as float4
  const int di = D.di, R = D.R, r = D.r;
  const int cl = threadIdx.x % TBK_CPB, k = threadIdx.x / TBK_CPB;
  float* s_delta = smem;                                                 // [TB][R]
  float* s_tok = smem + TB * (RB + 2 * DS) + cl * S::TSTR;               // [TB][4]
  float* s_h = smem + TB * (RB + 2 * DS) + TBK_CPB * S::TSTR + cl * S::CSTR;  // [TB][HS]
  const int base = blockIdx.x * TBK_CPB;
  const int b = base / di;
  const int c0 = base - b * di, c = c0 + cl;
  float* ssm = ssm_state + ((size_t)b * di + c) * DS + SPT * k;
  float h[SPT], na[SPT], wdt[RB];
#pragma unroll
  for (int n = 0; n < SPT; ++n) {
    h[n] = ssm[n];
    na[n] = Lw.na2[(size_t)c * DS + SPT * k + n];
  }
#pragma unroll
  for (int j = 0; j < RB; ++j) wdt[j] = j < r ? Lw.w_dt[(size_t)j * di + c] : 0.0f;
  const float bdt = Lw.b_dt[c], dd = Lw.dd[c];
  const TA* drows = delta + (size_t)b * T * R;
  const size_t row0 = (size_t)b * T;
  float pd[ND], pu[TPT], pz[TPT];
  auto fetch = [&](int t0) {
    const int nt = min(TB, T - t0);
#pragma unroll
    for (int i = 0; i < ND; ++i) {
      const int q = threadIdx.x + NT * i;
      pd[i] = q < nt * R ? ldv(drows + (size_t)t0 * R + q) : 0.0f;
    }
#pragma unroll
    for (int i = 0; i < TPT; ++i) {
      const int tok = k + G * i;
      const size_t row = row0 + t0 + tok;
      pu[i] = tok < nt ? ldv(conv + row * di + c) : 0.0f;
      pz[i] = tok < nt ? ldv(xz + row * 2 * di + di + c) : 0.0f;
    }
  };
  fetch(0);
  for (int t0 = 0; t0 < T; t0 += TB) {
    const int nt = min(TB, T - t0);
    __syncthreads();  // the previous pass no longer reads s_delta, s_tok, s_h
#pragma unroll
    for (int i = 0; i < ND; ++i) {
      const int q = threadIdx.x + NT * i;
      if (q < nt * R) s_delta[q] = pd[i];
    }
    float cu[TPT], cz[TPT];
#pragma unroll
    for (int i = 0; i < TPT; ++i) {
      cu[i] = pu[i];
      cz[i] = pz[i];
    }
    if (t0 + TB < T) fetch(t0 + TB);
    __syncthreads();
    // 1. the scalars of tokens k, k + 16, ...
#pragma unroll
    for (int i = 0; i < TPT; ++i) {
      const int tok = k + G * i;
      if (tok < nt) {
        const float* dv = s_delta + tok * R;
        float acc = 0.0f;
#pragma unroll
        for (int j = 0; j < RB; ++j)
          if (j < r) acc = __builtin_fmaf(dv[j], wdt[j], acc);
        const float dt = softplus<M>(acc + bdt);
        const float sg = rcp_sel<M>(1.0f + exp_sel<M>(-cz[i]));
        *reinterpret_cast<float4*>(s_tok + 4 * tok) =
            make_float4(dt, scan_fused_update<DS, M>() ? dt * cu[i] : cu[i], dd * cu[i], cz[i] * sg);
      }
    }
    __syncthreads();
    // 2. states SPT k .. SPT k + SPT - 1 through the pass's tokens
#pragma unroll 8
    for (int tt = 0; tt < nt; ++tt) {
      const float2 dd2 = *reinterpret_cast<const float2*>(s_tok + 4 * tt);
      const float* Bv = s_delta + tt * R + r;
#pragma unroll
      for (int n = 0; n < SPT; ++n) {
        const float dA = exp2_neg_sel<M>(na[n] * dd2.x);
        if constexpr (scan_fused_update<DS, M>()) {  // dd2.y = dt u
          h[n] = __builtin_fmaf(dA, h[n], Bv[SPT * k + n] * dd2.y);
        } else {  // dd2.y = u
          const float dB = dd2.x * Bv[SPT * k + n];
          h[n] = dA * h[n] + dB * dd2.y;
        }
        s_h[tt * HS + SPT * k + n] = h[n];
      }
    }
    __syncthreads();
    // 3. the outputs of tokens k, k + 16, ...
#pragma unroll
    for (int i = 0; i < TPT; ++i) {
      const int tok = k + G * i;
      if (tok < nt) {
        const float* Cv = s_delta + tok * R + r + DS;
        const float* hr = s_h + tok * HS;
        float yv = 0.0f;
#pragma unroll
        for (int n = 0; n < DS; ++n)
          yv = scan_fused_update<DS, M>() ? __builtin_fmaf(hr[n], Cv[n], yv) : yv + hr[n] * Cv[n];
        const float4 tk = *reinterpret_cast<const float4*>(s_tok + 4 * tok);
        yv = yv + tk.z;
        stv(y + (row0 + t0 + tok) * di + c, yv * tk.w);
      }
    }
  }
#pragma unroll
  for (int n = 0; n < SPT; ++n) ssm[n] = h[n];
}

static int block_for(int di) {
  for (int bs = 256; bs >= 32; bs >>= 1)
    if (di % bs == 0) return bs;
  return 0;
}

#ifndef BOA_SCAN_TBLK_BELOW
#define BOA_SCAN_TBLK_BELOW (64 * 1024)  // threads: one wave per SIMD
#endif

template <int DS, int RB>
static hipError_t scan_chunk_go(const Dims& D, const LayerW& Lw, const void* xz, const void* conv,
                                const void* delta, float* ssm_state, void* y, int lanes, int T,
                                int bs, bool bf16, hipStream_t s) {
  const dim3 grid((lanes * D.di) / bs);
  if ((int64_t)lanes * D.di < BOA_SCAN_TBLK_BELOW) {
    if (D.di % TBK_CPB) return hipErrorInvalidValue;
    const size_t lds = sizeof(float) * TblkShape<DS>::template lds_floats<RB>();
    const dim3 g2((lanes * D.di) / TBK_CPB);
    if (bf16)
      BOA_LAUNCH((scan_chunk_tblk_kernel<DS, RB, uint16_t>), g2, dim3(TBK_CPB * 16), lds, s, D,
                 Lw, (const uint16_t*)xz, (const uint16_t*)conv, (const uint16_t*)delta, ssm_state,
                 (uint16_t*)y, lanes, T);
    else
      BOA_LAUNCH((scan_chunk_tblk_kernel<DS, RB, float>), g2, dim3(TBK_CPB * 16), lds, s, D, Lw,
                 (const float*)xz, (const float*)conv, (const float*)delta, ssm_state, (float*)y,
                 lanes, T);
  } else if (bf16 && D.r == RB)
    BOA_LAUNCH((scan_chunk_sload_kernel<DS, RB, true, uint16_t>), grid, dim3(bs), 0, s, D, Lw,
               (const uint16_t*)xz, (const uint16_t*)conv, (const uint16_t*)delta, ssm_state,
               (uint16_t*)y, lanes, T);
  else if (bf16)
    BOA_LAUNCH((scan_chunk_sload_kernel<DS, RB, false, uint16_t>), grid, dim3(bs), 0, s, D, Lw,
               (const uint16_t*)xz, (const uint16_t*)conv, (const uint16_t*)delta, ssm_state,
               (uint16_t*)y, lanes, T);
  else if (D.r == RB)
    BOA_LAUNCH((scan_chunk_sload_kernel<DS, RB, true, float>), grid, dim3(bs), 0, s, D, Lw,
               (const float*)xz, (const float*)conv, (const float*)delta, ssm_state, (float*)y,
               lanes, T);
  else
    BOA_LAUNCH((scan_chunk_sload_kernel<DS, RB, false, float>), grid, dim3(bs), 0, s, D, Lw,
               (const float*)xz, (const float*)conv, (const float*)delta, ssm_state, (float*)y,
               lanes, T);
  return hipGetLastError();
}

// dt_rank bound RB in {8, 16, 32}: the smallest that holds D.r.
#define BOA_SCAN_DISPATCH(GO, ...)                                        \
  do {                                                                    \
    if (D.ds == 16) {                                                     \
      if (D.r <= 8) return GO<16, 8>(__VA_ARGS__);                        \
      if (D.r <= 16) return GO<16, 16>(__VA_ARGS__);                      \
      return GO<16, 32>(__VA_ARGS__);                                     \
    }                                                                     \
    if (D.r <= 8) return GO<32, 8>(__VA_ARGS__);                          \
    if (D.r <= 16) return GO<32, 16>(__VA_ARGS__);                        \
    return GO<32, 32>(__VA_ARGS__);                                       \
  } while (0)

hipError_t launch_scan_chunk(const Dims& D, const LayerW& Lw, const void* xz, const void* conv,
                             const void* delta, float* ssm_state, void* y, int lanes, int T,
                             bool bf16, hipStream_t s) {
  const int bs = block_for(D.di);
  if (!bs || D.r > RMAX || (D.ds != 16 && D.ds != 32)) return hipErrorInvalidValue;
  BOA_SCAN_DISPATCH(scan_chunk_go, D, Lw, xz, conv, delta, ssm_state, y, lanes, T, bs, bf16, s);
}

// ------------------------------------------------------------------ misc
__global__ void fill_zero_kernel(uint32_t* p, size_t n) {
  size_t i = (size_t)blockIdx.x * blockDim.x + threadIdx.x;
  size_t stride = (size_t)gridDim.x * blockDim.x;
  for (; i < n; i += stride) p[i] = 0u;
}

hipError_t launch_fill_zero(void* p, size_t bytes, hipStream_t s) {
  if (bytes % 4) return hipErrorInvalidValue;
  size_t n = bytes / 4;
  if (!n) return hipSuccess;
  size_t blocks = (n + 255) / 256;
  if (blocks > 65536) blocks = 65536;
  BOA_LAUNCH(fill_zero_kernel, dim3((unsigned)blocks), dim3(256), 0, s, (uint32_t*)p, n);
  return hipGetLastError();
}

}  // namespace boa
