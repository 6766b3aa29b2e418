// fp32 GEMM on CDNA4 matrix cores with the codec's fused epilogues.
//
//   C[m][n] = act(sum_k X[m][k] * W[k][n] + bias[n]) (+ R[m][n])
//
// Rounding contract (replaces gemm_kernels.cu:283-313 of the reference):
// every output is the K-ordered fused multiply-add chain acc = fma(x_k, w_k,
// acc) starting from 0, then `acc + bias` (0 when absent), then the
// activation, then `+ residual`.  v_mfma_f32_16x16x4_f32 on gfx950 evaluates
// its four products as exactly that sequential fma chain (k ascending), and
// the kernel issues the MFMAs of one output strictly in ascending k, never
// splitting K.  The result of an output row therefore does not depend on M,
// on the tile shape or on the row's position in the tile: the compress
// (M = lanes x tile) and decompress (M = lanes) passes produce bit-identical
// logits, and so does the CPU restatement that runs the same fma chain.
//
// Operand roles: the weight tile is the MFMA A operand (16 n-rows x 4 k) and
// the activation tile the B operand (4 k x 16 m-columns), so a lane's 4
// accumulators are 4 consecutive n of one row m and the epilogue stores a
// float4 per lane.  LDS: activations [BM][BK+4] (16-byte rows for b128
// stores), weights [BK][BN+16]; both double-buffered, one barrier per K step.
#include "boa_kernels.h"

namespace boa {

typedef float floatx4 __attribute__((ext_vector_type(4)));

template <int BM, int BN, int WAVES_M, int WAVES_N>
__global__ __launch_bounds__(64 * WAVES_M * WAVES_N) void gemm_f32_kernel(
    const float* __restrict__ X, int ldx, const float* __restrict__ W, int ldw, float* C, int ldc,
    const float* __restrict__ bias, const float* res, int ldr, int M, int N, int K, int act,
    int vec_store) {
  constexpr int BK = 16;
  constexpr int NT = 64 * WAVES_M * WAVES_N;
  constexpr int WM = BM / WAVES_M, WN = BN / WAVES_N;
  constexpr int TM = WM / 16, TN = WN / 16;
  constexpr int XS = BK + 4;   // activation row stride in LDS (floats)
  constexpr int WS = BN + 16;  // weight row stride in LDS (floats)
  constexpr int XL = BM * (BK / 4) / NT;  // float4 activation loads per thread
  constexpr int WL = BK * (BN / 4) / NT;  // float4 weight loads per thread
  static_assert(XL * NT == BM * (BK / 4), "activation tile load split");
  static_assert(WL * NT == BK * (BN / 4), "weight tile load split");
  __shared__ __attribute__((aligned(16))) float xs[2][BM * XS];
  __shared__ __attribute__((aligned(16))) float ws[2][BK * WS];

  const int tid = threadIdx.x;
  const int lane = tid & 63;
  const int wave = tid >> 6;
  const int wm0 = (wave / WAVES_N) * WM;
  const int wn0 = (wave % WAVES_N) * WN;
  const int g = lane >> 4, j = lane & 15;
  const int m_blk = blockIdx.y * BM, n_blk = blockIdx.x * BN;

  floatx4 acc[TM][TN];
#pragma unroll
  for (int a = 0; a < TM; ++a)
#pragma unroll
    for (int b = 0; b < TN; ++b) acc[a][b] = floatx4{0.f, 0.f, 0.f, 0.f};

  float4 xr[XL], wr[WL];
  auto load_tile = [&](int k0) {
#pragma unroll
    for (int i = 0; i < XL; ++i) {
      int q = tid + i * NT;
      int row = q / (BK / 4), k4 = q % (BK / 4);
      int gm = m_blk + row;
      gm = gm < M ? gm : M - 1;  // rows past M are computed but never stored
      xr[i] = *reinterpret_cast<const float4*>(X + (size_t)gm * ldx + k0 + 4 * k4);
    }
#pragma unroll
    for (int i = 0; i < WL; ++i) {
      int q = tid + i * NT;
      int kr = q / (BN / 4), n4 = q % (BN / 4);
      wr[i] = *reinterpret_cast<const float4*>(W + (size_t)(k0 + kr) * ldw + n_blk + 4 * n4);
    }
  };
  auto store_tile = [&](int buf) {
#pragma unroll
    for (int i = 0; i < XL; ++i) {
      int q = tid + i * NT;
      int row = q / (BK / 4), k4 = q % (BK / 4);
      *reinterpret_cast<float4*>(&xs[buf][row * XS + 4 * k4]) = xr[i];
    }
#pragma unroll
    for (int i = 0; i < WL; ++i) {
      int q = tid + i * NT;
      int kr = q / (BN / 4), n4 = q % (BN / 4);
      *reinterpret_cast<float4*>(&ws[buf][kr * WS + 4 * n4]) = wr[i];
    }
  };

  const int n_kt = K / BK;
  load_tile(0);
  store_tile(0);
  __syncthreads();
  for (int kt = 0; kt < n_kt; ++kt) {
    const int cur = kt & 1;
    if (kt + 1 < n_kt) load_tile((kt + 1) * BK);
#pragma unroll
    for (int kk = 0; kk < BK / 4; ++kk) {
      float af[TN], bf[TM];
#pragma unroll
      for (int b = 0; b < TN; ++b) af[b] = ws[cur][(kk * 4 + g) * WS + wn0 + b * 16 + j];
#pragma unroll
      for (int a = 0; a < TM; ++a) bf[a] = xs[cur][(wm0 + a * 16 + j) * XS + kk * 4 + g];
#pragma unroll
      for (int a = 0; a < TM; ++a)
#pragma unroll
        for (int b = 0; b < TN; ++b)
          acc[a][b] = __builtin_amdgcn_mfma_f32_16x16x4f32(af[b], bf[a], acc[a][b], 0, 0, 0);
    }
    if (kt + 1 < n_kt) store_tile(cur ^ 1);
    __syncthreads();
  }

  // Epilogue: lane owns C[m][n .. n+3], m = wm0 + a*16 + j, n = wn0 + b*16 + 4g.
#pragma unroll
  for (int a = 0; a < TM; ++a) {
    const int m = m_blk + wm0 + a * 16 + j;
    if (m >= M) continue;
#pragma unroll
    for (int b = 0; b < TN; ++b) {
      const int n = n_blk + wn0 + b * 16 + 4 * g;
      if (n >= N) continue;
      float v[4] = {acc[a][b][0], acc[a][b][1], acc[a][b][2], acc[a][b][3]};
#pragma unroll
      for (int e = 0; e < 4; ++e) {
        float t = v[e] + (bias ? bias[n + e < N ? n + e : N - 1] : 0.0f);
        if (act == ACT_GELU) t = gelu(t);
        else if (act == ACT_RELU) t = fmaxf(0.0f, t);
        v[e] = t;
      }
      if (vec_store) {
        if (res) {
          float4 r = *reinterpret_cast<const float4*>(res + (size_t)m * ldr + n);
          v[0] = v[0] + r.x; v[1] = v[1] + r.y; v[2] = v[2] + r.z; v[3] = v[3] + r.w;
        }
        *reinterpret_cast<float4*>(C + (size_t)m * ldc + n) = make_float4(v[0], v[1], v[2], v[3]);
      } else {
#pragma unroll
        for (int e = 0; e < 4; ++e) {
          if (n + e >= N) break;
          float t = v[e];
          if (res) t = t + res[(size_t)m * ldr + n + e];
          C[(size_t)m * ldc + n + e] = t;
        }
      }
    }
  }
}

template <int BM, int BN, int WM_, int WN_>
static hipError_t launch_cfg(const GemmArgs& a, hipStream_t s) {
  dim3 grid((a.N + BN - 1) / BN, (a.M + BM - 1) / BM);
  int vec = (a.N % 4 == 0) && (a.ldc % 4 == 0) && (!a.res || a.ldr % 4 == 0);
  hipLaunchKernelGGL((gemm_f32_kernel<BM, BN, WM_, WN_>), grid, dim3(64 * WM_ * WN_), 0, s, a.X,
                     a.ldx, a.W, a.ldw, a.C, a.ldc, a.bias, a.res, a.ldr, a.M, a.N, a.K, a.act,
                     vec);
  return hipGetLastError();
}

// Tile choice only changes the schedule, never the numerics (see above).
hipError_t gemm_f32(const GemmArgs& a, hipStream_t s) {
  if (a.M <= 0 || a.N <= 0) return hipSuccess;
  if (a.K % 16 != 0 || a.ldx % 4 != 0 || a.ldw % 4 != 0 || a.ldw < ((a.N + 127) / 128) * 128)
    return hipErrorInvalidValue;
  const long long tiles128 = (long long)((a.M + 127) / 128) * ((a.N + 127) / 128);
  if (a.N >= 128 && tiles128 >= 1024) return launch_cfg<128, 128, 2, 2>(a, s);
  const long long tiles64 = (long long)((a.M + 63) / 64) * ((a.N + 63) / 64);
  if (tiles64 >= 512) return launch_cfg<64, 64, 2, 2>(a, s);
  return launch_cfg<32, 64, 1, 2>(a, s);
}

}  // namespace boa
