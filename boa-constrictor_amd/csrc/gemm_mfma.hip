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
#include "coder_device.h"

namespace boa {

typedef float floatx4 __attribute__((ext_vector_type(4)));

// Epilogue mode of head.2 fused with the CDF (not a user activation): the
// block's logits rows go to LDS, and each row's (low, prob) pair of the
// next input byte is computed there (cdf_row_lowprob).
constexpr int ACT_CDF = 3;
// Epilogue modes of a 256-wide GEMM followed by a LayerNorm (see gemm_f32_ln).
constexpr int ACT_LN1 = 4, ACT_LN2 = 5;

// Eight waves per SIMD (64 VGPRs): two 16-wave blocks share a CU.
template <int BM, int BN, int WAVES_M, int WAVES_N, int BK, int ACT>
__global__ __launch_bounds__(64 * WAVES_M * WAVES_N) __attribute__((amdgpu_waves_per_eu(8, 8)))
void gemm_f32_kernel(
    const float* __restrict__ X, int ldx, const float* __restrict__ W, int ldw, float* C, int ldc,
    const float* __restrict__ bias, const float* res, int ldr, int M, int N, int K,
    int vec_store, int swizzle, CdfEpi cdf, LnEpi ln) {
  constexpr int NT = 64 * WAVES_M * WAVES_N;
  constexpr int WM = BM / WAVES_M, WN = BN / WAVES_N;
  constexpr int TM = WM / 16, TN = WN / 16;
  constexpr int XS = BK + 4;   // activation row stride in LDS (floats)
  constexpr int WS = BN + 16;  // weight row stride in LDS (floats)
  constexpr int XQ = BM * (BK / 4), WQ = BK * (BN / 4);  // float4s per tile
  constexpr int XL = (XQ + NT - 1) / NT;  // float4 activation loads per thread
  constexpr int WL = (WQ + NT - 1) / NT;  // float4 weight loads per thread
  // LDS: the K loop's double-buffered tiles; the CDF epilogue reuses the
  // same words for the block's logits rows (stride LS)
  constexpr int LS = BN + 4;
  constexpr int MAIN = 2 * BM * XS + 2 * BK * WS;
  constexpr int EPI = ACT == ACT_CDF ? BM * LS : ((ACT == ACT_LN1 || ACT == ACT_LN2) ? 64 * (BN + 3) : 0);
  __shared__ __attribute__((aligned(16))) float smem[MAIN > EPI ? MAIN : EPI];
  float(*xs)[BM * XS] = reinterpret_cast<float(*)[BM * XS]>(smem);
  float(*ws)[BK * WS] = reinterpret_cast<float(*)[BK * WS]>(smem + 2 * BM * XS);

  const int tid = threadIdx.x;
  const int lane = tid & 63;
  const int wave = tid >> 6;
  const int wm0 = (wave / WAVES_N) * WM;
  const int wn0 = (wave % WAVES_N) * WN;
  const int g = lane >> 4, j = lane & 15;
  // Workgroup w runs on XCD w % 8.  With the swizzle, each XCD gets a
  // contiguous range of tiles (all n-blocks of its m-blocks), so an activation
  // row-block is fetched into one XCD's L2 instead of into all eight.
  const int nb = (N + BN - 1) / BN;
  int w = blockIdx.x;
  if (swizzle) {
    const int total = gridDim.x, per = total / 8;
    if (w < per * 8) w = (w % 8) * per + w / 8;
  }
  const int m_blk = (w / nb) * BM, n_blk = (w % nb) * BN;

  floatx4 acc[TM][TN];
#pragma unroll
  for (int a = 0; a < TM; ++a)
#pragma unroll
    for (int b = 0; b < TN; ++b) acc[a][b] = floatx4{0.f, 0.f, 0.f, 0.f};

  // The block's bias values (clamped at N - 1) in LDS before the K loop, so
  // that the epilogue does not wait on global loads.
  __shared__ float sbias[BN];
  for (int c = tid; c < BN; c += NT) sbias[c] = bias ? bias[min(n_blk + c, N - 1)] : 0.0f;

  float4 xr[XL], wr[WL];
  auto load_tile = [&](int k0) {
#pragma unroll
    for (int i = 0; i < XL; ++i) {
      int q = tid + i * NT;
      if (XQ % NT && q >= XQ) break;
      int row = q / (BK / 4), k4 = q % (BK / 4);
      int gm = m_blk + row;
      gm = gm < M ? gm : M - 1;  // rows past M are computed but never stored
      xr[i] = *reinterpret_cast<const float4*>(X + (size_t)gm * ldx + k0 + 4 * k4);
    }
#pragma unroll
    for (int i = 0; i < WL; ++i) {
      int q = tid + i * NT;
      if (WQ % NT && q >= WQ) break;
      int kr = q / (BN / 4), n4 = q % (BN / 4);
      wr[i] = *reinterpret_cast<const float4*>(W + (size_t)(k0 + kr) * ldw + n_blk + 4 * n4);
    }
  };
  auto store_tile = [&](int buf) {
#pragma unroll
    for (int i = 0; i < XL; ++i) {
      int q = tid + i * NT;
      if (XQ % NT && q >= XQ) break;
      int row = q / (BK / 4), k4 = q % (BK / 4);
      *reinterpret_cast<float4*>(&xs[buf][row * XS + 4 * k4]) = xr[i];
    }
#pragma unroll
    for (int i = 0; i < WL; ++i) {
      int q = tid + i * NT;
      if (WQ % NT && q >= WQ) break;
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

  if constexpr (ACT == ACT_CDF) {
    // head.2 + bias into LDS (the K loop ended with a barrier, so the tile
    // buffers are free), then per row the CDF (cdf_row_lowprob)
    static_assert(BN == 256, "one block holds whole logits rows");
#pragma unroll
    for (int a = 0; a < TM; ++a)
#pragma unroll
      for (int b = 0; b < TN; ++b)
#pragma unroll
        for (int e = 0; e < 4; ++e) {
          const int col = wn0 + b * 16 + 4 * g + e;
          smem[(wm0 + a * 16 + j) * LS + col] = acc[a][b][e] + sbias[col];
        }
    __syncthreads();
    const int hw = tid >> 5, l = tid & 31;
    for (int r = hw; r < BM; r += NT / 32) cdf_row_lowprob(smem + r * LS, cdf, m_blk + r, M, l);
    return;
  }

  if constexpr (ACT == ACT_LN1 || ACT == ACT_LN2) {
    // Whole 256-feature rows in the block, 64 rows at a time through LDS
    // (the K loop ended with a barrier, so the tile buffers are free).  Row
    // stride RS = 257 keeps LN2's thread-per-row reads conflict-free; the
    // rows' statistics follow the 64 rows.
    static_assert(BN == 256 && BM == 128 && WAVES_M == 4, "64-row halves of whole rows");
    constexpr int D = 256, RS = D + 1;
    float* stat = smem + 64 * RS;
    for (int half = 0; half < 2; ++half) {
      if (wm0 / 64 == half) {
#pragma unroll
        for (int a = 0; a < TM; ++a) {
          const int rl = wm0 - 64 * half + a * 16 + j;
#pragma unroll
          for (int b = 0; b < TN; ++b) {
            const int n = wn0 + b * 16 + 4 * g;
#pragma unroll
            for (int e = 0; e < 4; ++e) smem[rl * RS + n + e] = acc[a][b][e] + sbias[n + e];
          }
        }
      }
      __syncthreads();
      if (ACT == ACT_LN1) {  // + residual; the sum is the residual stream's next value
#pragma unroll 1
        for (int it = 0; it < 4; ++it) {
          const int rl = (tid >> 6) + 16 * it, c = 4 * (tid & 63);
          const int m = m_blk + 64 * half + rl;
          if (m < M) {
            float* v = smem + rl * RS + c;
            const float4 r = *reinterpret_cast<const float4*>(res + (size_t)m * ldr + c);
            const float4 o = make_float4(v[0] + r.x, v[1] + r.y, v[2] + r.z, v[3] + r.w);
            *reinterpret_cast<float4*>(C + (size_t)m * ldc + c) = o;
            v[0] = o.x; v[1] = o.y; v[2] = o.z; v[3] = o.w;
          }
        }
        __syncthreads();
        // ln1_kernel's order: half-wave per row, lane l sums l, l+32, ...,
        // then the shuffle-down tree; lane 0 holds the totals
        const int hw = tid >> 5, l = tid & 31;
#pragma unroll
        for (int rr = 0; rr < 2; ++rr) {
          const int row_i = hw + 32 * rr;
          const float* row = smem + row_i * RS;
          float sm = 0.0f, sq = 0.0f;
#pragma unroll
          for (int e = 0; e < D / 32; ++e) {
            const float v = row[l + 32 * e];
            sm = sm + v;
            sq = sq + v * v;
          }
#pragma unroll
          for (int off = 16; off > 0; off >>= 1) {
            sm = sm + __shfl_down(sm, off, 32);
            sq = sq + __shfl_down(sq, off, 32);
          }
          if (l == 0) {
            const float mean = sm / (float)ln.n;
            const float var = sq / (float)ln.n - mean * mean;
            stat[2 * row_i] = mean;
            stat[2 * row_i + 1] = 1.0f / __builtin_sqrtf(var + 1e-5f);
          }
        }
      } else if (tid < 64) {  // ln2_kernel's order: one thread per row, elements in order
        const float* row = smem + tid * RS;
        float sm = 0.0f, sq = 0.0f;
        for (int i = 0; i < D; ++i) {
          const float e = row[i];
          sm = sm + e;
          sq = sq + e * e;
        }
        const float mean = sm / (float)ln.n;
        const float var = sq / (float)ln.n - mean * mean;
        stat[2 * tid] = mean;
        stat[2 * tid + 1] = 1.0f / __builtin_sqrtf(var + 1e-5f);
      }
      __syncthreads();
      // normalise: thread t takes columns 4(t % 64) .. +3 of rows t / 64 + 16i
#pragma unroll 1
      for (int it = 0; it < 4; ++it) {
        const int rl = (tid >> 6) + 16 * it, c = 4 * (tid & 63);
        const int m = m_blk + 64 * half + rl;
        const float mean = stat[2 * rl], inv_std = stat[2 * rl + 1];
        const float* v = smem + rl * RS + c;
        const float4 wv = *reinterpret_cast<const float4*>(ln.w + c);
        const float4 bv = *reinterpret_cast<const float4*>(ln.b + c);
        float4 o;
        o.x = ((v[0] - mean) * inv_std) * wv.x + bv.x;
        o.y = ((v[1] - mean) * inv_std) * wv.y + bv.y;
        o.z = ((v[2] - mean) * inv_std) * wv.z + bv.z;
        o.w = ((v[3] - mean) * inv_std) * wv.w + bv.w;
        if (m < M) *reinterpret_cast<float4*>(ln.out + (size_t)m * ln.ldo + c) = o;
      }
      __syncthreads();  // the next half reuses the rows
    }
    return;
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
        float t = v[e] + sbias[wn0 + b * 16 + 4 * g + e];
        if (ACT == ACT_GELU) t = gelu(t);
        else if (ACT == ACT_RELU) t = fmaxf(0.0f, t);
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

template <int BM, int BN, int WM_, int WN_, int BK>
static hipError_t launch_cfg(const GemmArgs& a, hipStream_t s, int swizzle = 1) {
  if (a.K % BK || a.ldw < (a.N + BN - 1) / BN * BN) return hipErrorInvalidValue;
  const long long tiles = (long long)((a.N + BN - 1) / BN) * ((a.M + BM - 1) / BM);
  if (tiles >= (1ll << 31)) return hipErrorInvalidValue;
  int vec = (a.N % 4 == 0) && (a.ldc % 4 == 0) && (!a.res || a.ldr % 4 == 0);
  // the activation is a template argument: the epilogue has no branch on it
#define BOA_GEMM_GO(ACTv)                                                                     \
  BOA_LAUNCH((gemm_f32_kernel<BM, BN, WM_, WN_, BK, ACTv>), dim3((unsigned)tiles),     \
                     dim3(64 * WM_ * WN_), 0, s, a.X, a.ldx, a.W, a.ldw, a.C, a.ldc, a.bias,   \
                     a.res, a.ldr, a.M, a.N, a.K, vec, swizzle, CdfEpi{}, LnEpi{})
  switch (a.act) {
    case ACT_NONE: BOA_GEMM_GO(ACT_NONE); break;
    case ACT_GELU: BOA_GEMM_GO(ACT_GELU); break;
    case ACT_RELU: BOA_GEMM_GO(ACT_RELU); break;
    default: return hipErrorInvalidValue;
  }
#undef BOA_GEMM_GO
  return hipGetLastError();
}

// Tile choice only changes the schedule, never the numerics (see above).
// Chosen from a sweep on MI355X (fp32 MFMA): many waves per CU matter more
// than register blocking.  Large M (a compress tile): 128x256 with 16 waves
// (32x64 each) for N >= 256, 128x64 with 8 waves for the narrow x_proj;
// small M (a decode step, M = lanes): 32x32 with four 16x16 waves and BK=32.
int gemm_f32_config(const GemmArgs& a) {
  if (a.M >= 16384) return a.N >= 256 ? 0 : 1;
  return 2;
}

// head.2 of a compress tile fused with the CDF: rows of 256 logits (acc +
// bias) stay in LDS and each row's (low, prob) of the next byte is written
// to cdf.lowprob.  64-row blocks keep two blocks per CU (66.5 KB of LDS).
hipError_t gemm_f32_head_cdf(const GemmArgs& a, const CdfEpi& cdf, hipStream_t s) {
  if (a.M <= 0) return hipSuccess;
  if (a.N != 256 || a.K % 16 || a.ldx % 4 || a.ldw % 4 || !cdf.lowprob || cdf.T < 1)
    return hipErrorInvalidValue;
  constexpr int BM = 64, BN = 256;  // 128-row blocks (one per CU) measured the same
  if (a.ldw < BN) return hipErrorInvalidValue;
  const long long tiles = (a.M + BM - 1) / BM;
  if (tiles >= (1ll << 31)) return hipErrorInvalidValue;
  BOA_LAUNCH((gemm_f32_kernel<BM, BN, 4, 4, 16, ACT_CDF>), dim3((unsigned)tiles), dim3(1024),
                     0, s, a.X, a.ldx, a.W, a.ldw, nullptr, 0, a.bias, nullptr, 0, a.M, a.N, a.K,
                     0, 1, cdf, LnEpi{});
  return hipGetLastError();
}

hipError_t gemm_f32_ln(const GemmArgs& a, const LnEpi& ln, hipStream_t s) {
  if (a.M <= 0) return hipSuccess;
  if (a.N != 256 || a.K % 16 || a.ldx % 4 || a.ldw < 256 || a.ldw % 4 || !ln.out || !ln.w ||
      !ln.b || ln.ldo % 4 || ln.ldo < 256 || (ln.mode == 1 && (!a.res || !a.C || a.ldr % 4 ||
      a.ldc % 4)))
    return hipErrorInvalidValue;
  const long long tiles = (a.M + 127) / 128;
  if (tiles >= (1ll << 31)) return hipErrorInvalidValue;
  if (ln.mode == 1)
    BOA_LAUNCH((gemm_f32_kernel<128, 256, 4, 4, 16, ACT_LN1>), dim3((unsigned)tiles), dim3(1024),
               0, s, a.X, a.ldx, a.W, a.ldw, a.C, a.ldc, a.bias, a.res, a.ldr, a.M, a.N, a.K, 1, 1,
               CdfEpi{}, ln);
  else if (ln.mode == 2)
    BOA_LAUNCH((gemm_f32_kernel<128, 256, 4, 4, 16, ACT_LN2>), dim3((unsigned)tiles), dim3(1024),
               0, s, a.X, a.ldx, a.W, a.ldw, a.C, a.ldc, a.bias, a.res, a.ldr, a.M, a.N, a.K, 1, 1,
               CdfEpi{}, ln);
  else
    return hipErrorInvalidValue;
  return hipGetLastError();
}

hipError_t gemm_f32(const GemmArgs& a, hipStream_t s) {
  if (a.M <= 0 || a.N <= 0) return hipSuccess;
  if (a.K % 16 != 0 || a.ldx % 4 != 0 || a.ldw % 4 != 0) return hipErrorInvalidValue;
  switch (gemm_f32_config(a)) {
    case 0: return launch_cfg<128, 256, 4, 4, 16>(a, s);
    case 1: return launch_cfg<128, 64, 4, 2, 16>(a, s);
    default:
      return a.K % 32 == 0 ? launch_cfg<32, 32, 2, 2, 32>(a, s) : launch_cfg<32, 32, 2, 2, 16>(a, s);
  }
}

}  // namespace boa
