// bf16 GEMM on CDNA4 matrix cores with the codec's fused epilogues:
//
//   C[m][n] = act(sum_k X[m][k] * W[n][k] + bias[n]) (+ R[m][n])
//
// X and W are bf16; accumulation is fp32 in v_mfma_f32_16x16x32_bf16.  W is
// stored n-major ([N_pad][K], k contiguous) so that both operands of an MFMA
// are 16-byte rows.  Every output is the chain of MFMAs over k-steps of 32 in
// ascending order from 0, with k = 32 s + 8 g + e in operand slot (g, e) of
// lane (i, g); the decode-step GEMM issues the same chain, so the compress and
// decompress passes produce identical logits.  The epilogue (bias, activation,
// residual) is the fp32 one; the output is stored in fp32 or bf16, and the
// last layer's FF2 can also store a bf16 copy of its fp32 output (head1's
// input).
//
// Operand roles as in the fp32 kernel: weights are the A operand (16 n-rows),
// activations the B operand (16 m-columns); a lane's accumulators are 4
// consecutive n of one row m.  LDS: [rows][BK + 8] u16 per operand (the pad
// staggers 16-byte row reads across banks), double-buffered.
#include "boa_kernels.h"

namespace boa {

typedef float floatx4 __attribute__((ext_vector_type(4)));
typedef uint32_t u32x4 __attribute__((ext_vector_type(4)));
typedef __bf16 bf16x8 __attribute__((ext_vector_type(8)));

// Epilogue of one tile: lane owns C[m][n .. n+3], m = m_blk + wm0 + 16p + j,
// n = n_blk + wn0 + 16q + 4g.  `sbias` holds the block's bias values
// (column c of the block at c, clamped at N - 1); the activation is a
// template argument, so the epilogue has no branch on it.
template <int TM, int TN, int ACT>
__device__ __forceinline__ void b16_epilogue(const GemmB16Args& a, const floatx4 (&acc)[TM][TN],
                                             int m_blk, int n_blk, int wm0, int wn0, int j, int g,
                                             const float* sbias) {
  const bool res4 = a.res && (a.ldr & 3) == 0;
#pragma unroll
  for (int p = 0; p < TM; ++p) {
    const int m = m_blk + wm0 + 16 * p + j;
    if (m >= a.M) continue;
#pragma unroll
    for (int q = 0; q < TN; ++q) {
      const int n = n_blk + wn0 + 16 * q + 4 * g;
      if (n >= a.N) continue;
      float rv[4] = {0.0f, 0.0f, 0.0f, 0.0f};
      if (res4 && n + 4 <= a.N) {
        const float4 t = *reinterpret_cast<const float4*>(a.res + (size_t)m * a.ldr + n);
        rv[0] = t.x; rv[1] = t.y; rv[2] = t.z; rv[3] = t.w;
      } else if (a.res) {
#pragma unroll
        for (int e = 0; e < 4; ++e) rv[e] = n + e < a.N ? a.res[(size_t)m * a.ldr + n + e] : 0.0f;
      }
      float v[4];
#pragma unroll
      for (int e = 0; e < 4; ++e) {
        float t = acc[p][q][e] + sbias[n - n_blk + e];
        if (ACT == ACT_GELU) t = gelu<MATH_HW>(t);
        else if (ACT == ACT_RELU) t = fmaxf(0.0f, t);
        if (a.res) t = t + rv[e];
        v[e] = t;
      }
      const size_t o = (size_t)m * a.ldc + n;
      if (n + 4 <= a.N) {
        if (a.c_bf16)
          *reinterpret_cast<ushort4*>(reinterpret_cast<uint16_t*>(a.C) + o) =
              make_ushort4(f32_to_bf16(v[0]), f32_to_bf16(v[1]), f32_to_bf16(v[2]), f32_to_bf16(v[3]));
        else
          *reinterpret_cast<float4*>(reinterpret_cast<float*>(a.C) + o) =
              make_float4(v[0], v[1], v[2], v[3]);
        if (a.C2)
          *reinterpret_cast<ushort4*>(a.C2 + o) =
              make_ushort4(f32_to_bf16(v[0]), f32_to_bf16(v[1]), f32_to_bf16(v[2]), f32_to_bf16(v[3]));
      } else {
#pragma unroll
        for (int e = 0; e < 4; ++e) {
          if (n + e >= a.N) break;
          if (a.c_bf16) reinterpret_cast<uint16_t*>(a.C)[o + e] = f32_to_bf16(v[e]);
          else reinterpret_cast<float*>(a.C)[o + e] = v[e];
          if (a.C2) a.C2[o + e] = f32_to_bf16(v[e]);
        }
      }
    }
  }
}

template <int BM, int BN, int WAVES_M, int WAVES_N, int BK, int NBUF, int ACT>
__global__ __launch_bounds__(64 * WAVES_M * WAVES_N) void gemm_bf16_kernel(GemmB16Args a,
                                                                           int swizzle) {
  constexpr int NT = 64 * WAVES_M * WAVES_N;
  constexpr int WM = BM / WAVES_M, WN = BN / WAVES_N;
  constexpr int TM = WM / 16, TN = WN / 16;
  constexpr int S = BK + 8;                          // LDS row stride (u16)
  constexpr int XQ = BM * BK / 8, WQ = BN * BK / 8;  // 16-byte chunks per tile
  constexpr int XL = (XQ + NT - 1) / NT, WL = (WQ + NT - 1) / NT;
  static_assert(BK % 32 == 0, "BK must be a multiple of the MFMA k-step");
  // NBUF = 1 keeps one LDS stage (the next k-tile waits in registers), so
  // two workgroups fit in a CU's LDS and one's epilogue overlaps the
  // other's main loop.
  __shared__ __attribute__((aligned(16))) uint16_t xs[NBUF][BM * S];
  __shared__ __attribute__((aligned(16))) uint16_t ws[NBUF][BN * S];
  __shared__ float sbias[BN];  // the block's bias values, for the epilogue

  const int tid = threadIdx.x;
  const int lane = tid & 63, wave = tid >> 6;
  const int wm0 = (wave / WAVES_N) * WM, wn0 = (wave % WAVES_N) * WN;
  const int g = lane >> 4, j = lane & 15;
  // workgroup w runs on XCD w % 8; the swizzle gives each XCD a contiguous
  // range of tiles so an activation row-block stays in one XCD's L2
  const int nb = (a.N + BN - 1) / BN;
  int w = blockIdx.x;
  if (swizzle) {
    const int total = gridDim.x, per = total / 8;
    if (w < per * 8) w = (w % 8) * per + w / 8;
  }
  const int m_blk = (w / nb) * BM, n_blk = (w % nb) * BN;
  for (int c = tid; c < BN; c += NT) sbias[c] = a.bias ? a.bias[min(n_blk + c, a.N - 1)] : 0.0f;

  floatx4 acc[TM][TN];
#pragma unroll
  for (int p = 0; p < TM; ++p)
#pragma unroll
    for (int q = 0; q < TN; ++q) acc[p][q] = floatx4{0.f, 0.f, 0.f, 0.f};

  u32x4 xr[XL], wr[WL];
#define BOA_B16_LOAD(K0)                                                               \
  _Pragma("unroll") for (int i = 0; i < XL; ++i) {                                     \
    const int q = tid + i * NT;                                                        \
    if (XQ % NT == 0 || q < XQ) {                                                      \
      const int row = q / (BK / 8), c8 = q % (BK / 8);                                 \
      const int gm = min(m_blk + row, a.M - 1);                                        \
      xr[i] = *reinterpret_cast<const u32x4*>(a.X + (size_t)gm * a.ldx + (K0) + 8 * c8); \
    }                                                                                  \
  }                                                                                    \
  _Pragma("unroll") for (int i = 0; i < WL; ++i) {                                     \
    const int q = tid + i * NT;                                                        \
    if (WQ % NT == 0 || q < WQ) {                                                      \
      const int row = q / (BK / 8), c8 = q % (BK / 8);                                 \
      wr[i] = *reinterpret_cast<const u32x4*>(a.W + (size_t)(n_blk + row) * a.ldw + (K0) + 8 * c8); \
    }                                                                                  \
  }
#define BOA_B16_STORE(BUF)                                                             \
  _Pragma("unroll") for (int i = 0; i < XL; ++i) {                                     \
    const int q = tid + i * NT;                                                        \
    if (XQ % NT == 0 || q < XQ)                                                        \
      *reinterpret_cast<u32x4*>(&xs[BUF][(q / (BK / 8)) * S + 8 * (q % (BK / 8))]) = xr[i]; \
  }                                                                                    \
  _Pragma("unroll") for (int i = 0; i < WL; ++i) {                                     \
    const int q = tid + i * NT;                                                        \
    if (WQ % NT == 0 || q < WQ)                                                        \
      *reinterpret_cast<u32x4*>(&ws[BUF][(q / (BK / 8)) * S + 8 * (q % (BK / 8))]) = wr[i]; \
  }

  const int n_kt = a.K / BK;
  BOA_B16_LOAD(0)
  BOA_B16_STORE(0)
  __syncthreads();
  for (int kt = 0; kt < n_kt; ++kt) {
    const int cur = NBUF == 2 ? (kt & 1) : 0;
    if (kt + 1 < n_kt) { BOA_B16_LOAD((kt + 1) * BK) }
#pragma unroll
    for (int ks = 0; ks < BK / 32; ++ks) {
      bf16x8 af[TN], bf[TM];
#pragma unroll
      for (int q = 0; q < TN; ++q)
        af[q] = __builtin_bit_cast(bf16x8, *reinterpret_cast<const u32x4*>(
                                               &ws[cur][(wn0 + 16 * q + j) * S + 32 * ks + 8 * g]));
#pragma unroll
      for (int p = 0; p < TM; ++p)
        bf[p] = __builtin_bit_cast(bf16x8, *reinterpret_cast<const u32x4*>(
                                               &xs[cur][(wm0 + 16 * p + j) * S + 32 * ks + 8 * g]));
#pragma unroll
      for (int p = 0; p < TM; ++p)
#pragma unroll
        for (int q = 0; q < TN; ++q)
          acc[p][q] = __builtin_amdgcn_mfma_f32_16x16x32_bf16(af[q], bf[p], acc[p][q], 0, 0, 0);
    }
    if (NBUF == 1 && kt + 1 < n_kt) __syncthreads();
    if (kt + 1 < n_kt) { BOA_B16_STORE(NBUF == 2 ? (cur ^ 1) : 0) }
    __syncthreads();
  }
#undef BOA_B16_LOAD
#undef BOA_B16_STORE

  b16_epilogue<TM, TN, ACT>(a, acc, m_blk, n_blk, wm0, wn0, j, g, sbias);
}

template <int BM, int BN, int WM_, int WN_, int BK, int NBUF = 2>
static hipError_t launch_b16(const GemmB16Args& a, hipStream_t s, int swizzle = 1) {
  if (a.K % BK || a.ldx % 8 || a.ldw % 8 || a.ldw < a.K) return hipErrorInvalidValue;
  const long long tiles = (long long)((a.N + BN - 1) / BN) * ((a.M + BM - 1) / BM);
  if (tiles >= (1ll << 31)) return hipErrorInvalidValue;
#define BOA_B16_GO(ACTv)                                                                  \
  BOA_LAUNCH((gemm_bf16_kernel<BM, BN, WM_, WN_, BK, NBUF, ACTv>), dim3((unsigned)tiles), \
                     dim3(64 * WM_ * WN_), 0, s, a, swizzle)
  switch (a.act) {
    case ACT_NONE: BOA_B16_GO(ACT_NONE); break;
    case ACT_GELU: BOA_B16_GO(ACT_GELU); break;
    case ACT_RELU: BOA_B16_GO(ACT_RELU); break;
    default: return hipErrorInvalidValue;
  }
#undef BOA_B16_GO
  return hipGetLastError();
}

// W must hold round_up(N, 256) rows (zero padded) for every configuration.
// Chosen from sweeps on MI355X at compress shapes (M ~ 10^6): 256x256 with
// 16 waves of 64x64 (the LDS traffic per MFMA halves against 32x64 waves) for
// N >= 256 -- one LDS stage where K or N is at least 512 (3-8 % faster
// there), two for the 256x256 head GEMMs -- and 128x64 with 8 waves for the
// narrow x_proj.  Smaller tiles (128x128, 8-wave 256x256) were 25-45 %
// slower.
hipError_t gemm_bf16(const GemmB16Args& a, hipStream_t s) {
  if (a.M <= 0 || a.N <= 0) return hipSuccess;
  if (a.N >= 256 && (a.N >= 512 || a.K >= 512)) return launch_b16<256, 256, 4, 4, 64, 1>(a, s);
  if (a.N >= 256) return launch_b16<256, 256, 4, 4, 64>(a, s);
  return launch_b16<128, 64, 4, 2, 64>(a, s);
}

// Weight relayout for the bf16 compress GEMM: W [K][ldw_in] fp32 (the fp32
// compress layout) -> [n_pad][K] bf16, rows n >= N zero.
__global__ void b16_weight_nk_kernel(const float* __restrict__ w, int ldw_in, int N, int K,
                                     int n_pad, uint16_t* out) {
  const size_t idx = (size_t)blockIdx.x * blockDim.x + threadIdx.x;
  if (idx >= (size_t)n_pad * K) return;
  const int n = (int)(idx / K), k = (int)(idx % K);
  out[idx] = n < N ? f32_to_bf16(w[(size_t)k * ldw_in + n]) : (uint16_t)0;
}

hipError_t launch_b16_weight_nk(const float* w, int ldw_in, int N, int K, int n_pad, uint16_t* out,
                                hipStream_t s) {
  if (n_pad < N || N > ldw_in) return hipErrorInvalidValue;
  const size_t n = (size_t)n_pad * K;
  BOA_LAUNCH(b16_weight_nk_kernel, dim3((unsigned)((n + 255) / 256)), dim3(256), 0, s, w,
                     ldw_in, N, K, n_pad, out);
  return hipGetLastError();
}

}  // namespace boa
