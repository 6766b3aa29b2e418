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
#include "coder_device.h"

namespace boa {

typedef float floatx4 __attribute__((ext_vector_type(4)));

// Epilogue mode of head.2 fused with the CDF (not a user activation): the
// block's logits rows pass through LDS 64 at a time and each row's (low,
// prob) pair of the next input byte is computed there (cdf_row_lowprob); the
// logits never reach memory.
constexpr int ACT_CDF = 3;
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
                                                                           int swizzle,
                                                                           CdfEpi cdf) {
  constexpr int NT = 64 * WAVES_M * WAVES_N;
  constexpr int WM = BM / WAVES_M, WN = BN / WAVES_N;
  constexpr int TM = WM / 16, TN = WN / 16;
  constexpr int S = BK + 8;                          // LDS row stride (u16)
  constexpr int XQ = BM * BK / 8, WQ = BN * BK / 8;  // 16-byte chunks per tile
  constexpr int XL = (XQ + NT - 1) / NT, WL = (WQ + NT - 1) / NT;
  static_assert(BK % 32 == 0, "BK must be a multiple of the MFMA k-step");
  // NBUF = 1 keeps one LDS stage (the next k-tile waits in registers), so
  // two workgroups fit in a CU's LDS and one's epilogue overlaps the
  // other's main loop.  The CDF epilogue reuses the words for 64 logits
  // rows of LS floats.
  constexpr int LS = BN + 4;
  constexpr int MAIN_B = NBUF * (BM + BN) * S * 2;
  constexpr int EPI_B = ACT == ACT_CDF ? 64 * LS * 4 : 0;
  __shared__ __attribute__((aligned(16))) uint16_t smem[(MAIN_B > EPI_B ? MAIN_B : EPI_B) / 2];
  uint16_t(*xs)[BM * S] = reinterpret_cast<uint16_t(*)[BM * S]>(smem);
  uint16_t(*ws)[BN * S] = reinterpret_cast<uint16_t(*)[BN * S]>(smem + NBUF * BM * S);
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

  if constexpr (ACT == ACT_CDF) {
    // the logits rows, acc + bias as the unfused epilogue stores them,
    // 64 rows (one wave row of the block) at a time; the K loop ended with
    // a barrier, so its buffers are free
    static_assert(BN == 256 && WM == 64, "whole logits rows, 64 per wave row");
    float* lg = reinterpret_cast<float*>(smem);
    const int hw = tid >> 5, l = tid & 31;
    for (int h = 0; h < BM / 64; ++h) {
      if (wm0 == 64 * h) {
#pragma unroll
        for (int p = 0; p < TM; ++p)
#pragma unroll
          for (int q = 0; q < TN; ++q)
#pragma unroll
            for (int e = 0; e < 4; ++e) {
              const int col = wn0 + 16 * q + 4 * g + e;
              lg[(16 * p + j) * LS + col] = acc[p][q][e] + sbias[col];
            }
      }
      __syncthreads();
      for (int r = hw; r < 64; r += NT / 32)
        cdf_row_lowprob(lg + r * LS, cdf, m_blk + 64 * h + r, a.M, l);
      __syncthreads();  // the next 64 rows reuse the buffer
    }
    return;
  }
  b16_epilogue<TM, TN, ACT>(a, acc, m_blk, n_blk, wm0, wn0, j, g, sbias);
}

template <int BM, int BN, int WM_, int WN_, int BK, int NBUF = 2>
static hipError_t launch_b16(const GemmB16Args& a, hipStream_t s, int swizzle = 1,
                             const CdfEpi* cdf = nullptr) {
  if (a.K % BK || a.ldx % 8 || a.ldw % 8 || a.ldw < a.K) return hipErrorInvalidValue;
  const long long tiles = (long long)((a.N + BN - 1) / BN) * ((a.M + BM - 1) / BM);
  if (tiles >= (1ll << 31)) return hipErrorInvalidValue;
  const CdfEpi ce = cdf ? *cdf : CdfEpi{};
#define BOA_B16_GO(ACTv)                                                                  \
  BOA_LAUNCH((gemm_bf16_kernel<BM, BN, WM_, WN_, BK, NBUF, ACTv>), dim3((unsigned)tiles), \
                     dim3(64 * WM_ * WN_), 0, s, a, swizzle, ce)
  if (cdf) {
    if constexpr (BN == 256 && BM / WM_ == 64) {
      if (a.N != 256 || a.act != ACT_NONE) return hipErrorInvalidValue;
      BOA_B16_GO(ACT_CDF);
      return hipGetLastError();
    } else {
      return hipErrorInvalidValue;
    }
  }
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

// head.2 (N = 256) fused with the CDF: the head GEMM's tile and stages, the
// epilogue of ACT_CDF; writes cdf.lowprob instead of the logits
hipError_t gemm_bf16_head_cdf(const GemmB16Args& a, const CdfEpi& cdf, hipStream_t s) {
  if (a.M <= 0) return hipSuccess;
  if (a.K >= 512) return launch_b16<256, 256, 4, 4, 64, 1>(a, s, 1, &cdf);
  return launch_b16<256, 256, 4, 4, 64>(a, s, 1, &cdf);
}

// ------------------------------------------------------ FF1 + GELU + FF2
// The feed-forward pair in one kernel: a block of 1024 threads owns BM rows
// and keeps their FF2 accumulators (BM x D fp32) in registers while the
// hidden layer passes through LDS HC columns at a time:
//   h = bf16(gelu(x . W1[c]^T + b1[c]))   (HC hidden columns of chunk c)
//   acc += h . W2[:, c]^T
// then acc + b2 + residual.  The hidden layer (4 D bf16 per row) never
// reaches HBM.  Every MFMA chain is the unfused GEMMs' (k-steps of 32 in
// ascending order from 0, k = 32 s + 8 g + e in operand slot (g, e); FF2's
// chain continues from chunk to chunk), and both epilogues are theirs, so
// the bits are those of gemm_bf16(FF1, GELU) + gemm_bf16(FF2).
// LDS rows are K-contiguous bf16 with 8 elements of padding.
// LNF bit 1: the block's rows of X are out_proj's output and LN2 runs on them
// in LDS before FF1, in ln2_kernel's order (one thread per row, elements in
// order, statistics from the bf16 values) and with its bf16 rounding of the
// result.  LNF bit 2: the fp32 output rows also pass through LDS, where the
// next layer's LN1 runs in ln1_kernel's order (half-wave per row, the
// 32-lane tree) and stores xn in bf16.
template <int D, int BM, int HC, int WM2, int WN2, int WM1, int WN1, int LNF>
__global__ __launch_bounds__(1024) void ffn_bf16_kernel(FfnB16Args a) {
  constexpr int H = 4 * D;
  // Row strides (bf16) of the LDS tiles.  The bank conflicts measured on
  // MI355X fit 16-byte fragment reads served 32 lanes at a time (16 rows j,
  // two 16-byte column groups g) over 128 four-byte banks: a row stride of
  // 8 mod 128 words (D + 16 bf16 at D = 256) puts those 32 reads on
  // distinct banks, while D + 8 (4 mod 128 words) paired them up.  C3
  // probe: FFN bank-conflict cycles 21.6 -> 8.9 % of its active cycles,
  // compress 19.32 -> 19.81 MB/s.  HP keeps HC + 8 (the tiles fill the LDS).
  constexpr int XP = D + 16, HP = HC + 8;
  constexpr int NC = H / HC;
  constexpr int TM2 = BM / WM2 / 16, TN2 = D / WN2 / 16;    // FF2 tiles per wave
  constexpr int TM1 = BM / WM1 / 16, TN1 = HC / WN1 / 16;   // FF1 tiles per wave
  static_assert(WM2 * WN2 == 16 && WM1 * WN1 <= 16, "16 waves");
  static_assert(TM2 >= 1 && TN2 >= 1 && TM1 >= 1 && TN1 >= 1, "tile shapes");
  constexpr int XQ = BM * D / 8, W1Q = HC * D / 8, W2Q = D * HC / 8;  // 16-byte chunks
  constexpr int XL = (XQ + 1023) / 1024, W1L = (W1Q + 1023) / 1024, W2L = (W2Q + 1023) / 1024;
  // one LDS buffer: the K loop's xs, w1s, hs, w2s; after it, the LN1
  // epilogue's fp32 rows (stride RS)
  constexpr int XS_B = BM * XP * 2, W1S_B = HC * XP * 2, HS_B = BM * HP * 2, W2S_B = D * HP * 2;
  constexpr int MAIN_B = XS_B + W1S_B + HS_B + W2S_B;
  constexpr int RS = D + 4;
  constexpr int EPI_B = (LNF & 2) ? BM * RS * 4 : 0;
  static_assert(XS_B % 16 == 0 && W1S_B % 16 == 0 && HS_B % 16 == 0, "16-byte aligned parts");
  __shared__ __attribute__((aligned(16))) unsigned char smem[MAIN_B > EPI_B ? MAIN_B : EPI_B];
  uint16_t* const xs = reinterpret_cast<uint16_t*>(smem);
  uint16_t* const w1s = reinterpret_cast<uint16_t*>(smem + XS_B);
  uint16_t* const hs = reinterpret_cast<uint16_t*>(smem + XS_B + W1S_B);
  uint16_t* const w2s = reinterpret_cast<uint16_t*>(smem + XS_B + W1S_B + HS_B);
  __shared__ float b1s[HC], b2s[D];
  __shared__ float lnst[2 * BM];  // LN2: per-row (mean, 1 / std)

  const int tid = threadIdx.x, lane = tid & 63, wave = tid >> 6;
  const int g = lane >> 4, j = lane & 15;
  const int m_blk = blockIdx.x * BM;

  // the block's rows and b2
#pragma unroll
  for (int it = 0; it < XL; ++it) {
    const int q = tid + it * 1024;
    if (XQ % 1024 == 0 || q < XQ) {
      const int row = q / (D / 8), c8 = q % (D / 8);
      const int gm = min(m_blk + row, a.M - 1);
      *reinterpret_cast<u32x4*>(&xs[row * XP + 8 * c8]) =
          *reinterpret_cast<const u32x4*>(a.X + (size_t)gm * D + 8 * c8);
    }
  }
  for (int c = tid; c < D; c += 1024) b2s[c] = a.b2 ? a.b2[c] : 0.0f;

  u32x4 w1r[W1L], w2r[W2L];
  float b1r = 0.0f;
  auto load_chunk = [&](int ch) {
#pragma unroll
    for (int it = 0; it < W1L; ++it) {
      const int q = tid + it * 1024;
      if (W1Q % 1024 == 0 || q < W1Q) {
        const int row = q / (D / 8), c8 = q % (D / 8);
        w1r[it] = *reinterpret_cast<const u32x4*>(a.W1 + (size_t)(ch * HC + row) * D + 8 * c8);
      }
    }
#pragma unroll
    for (int it = 0; it < W2L; ++it) {
      const int q = tid + it * 1024;
      if (W2Q % 1024 == 0 || q < W2Q) {
        const int row = q / (HC / 8), c8 = q % (HC / 8);
        w2r[it] = *reinterpret_cast<const u32x4*>(a.W2 + (size_t)row * H + ch * HC + 8 * c8);
      }
    }
    if (tid < HC) b1r = a.b1 ? a.b1[ch * HC + tid] : 0.0f;
  };
  auto store_chunk = [&]() {
#pragma unroll
    for (int it = 0; it < W1L; ++it) {
      const int q = tid + it * 1024;
      if (W1Q % 1024 == 0 || q < W1Q)
        *reinterpret_cast<u32x4*>(&w1s[(q / (D / 8)) * XP + 8 * (q % (D / 8))]) = w1r[it];
    }
#pragma unroll
    for (int it = 0; it < W2L; ++it) {
      const int q = tid + it * 1024;
      if (W2Q % 1024 == 0 || q < W2Q)
        *reinterpret_cast<u32x4*>(&w2s[(q / (HC / 8)) * HP + 8 * (q % (HC / 8))]) = w2r[it];
    }
    if (tid < HC) b1s[tid] = b1r;
  };

  // FF2 accumulators: wave (wm2, wn2) owns rows 16 TM2 wm2 + 16 p + j, features
  // 16 TN2 wn2 + 16 q + 4 g + v
  const int wm2 = wave / WN2, wn2 = wave % WN2;
  const int wm1 = wave / WN1, wn1 = wave % WN1;
  const bool ff1_wave = wave < WM1 * WN1;
  floatx4 acc2[TM2][TN2];
#pragma unroll
  for (int p = 0; p < TM2; ++p)
#pragma unroll
    for (int q = 0; q < TN2; ++q) acc2[p][q] = floatx4{0.f, 0.f, 0.f, 0.f};

  load_chunk(0);
  if constexpr ((LNF & 1) != 0) {
    // LN2 in place in xs while chunk 0's weights load (splitting the sums
    // and the sums of squares over two waves measured the same)
    __syncthreads();
    if (tid < BM) {
      const uint16_t* row = xs + tid * XP;
      float sm = 0.0f, sq = 0.0f;
      for (int c8 = 0; c8 < D / 8; ++c8) {
        const u32x4 w = *reinterpret_cast<const u32x4*>(row + 8 * c8);
#pragma unroll
        for (int e = 0; e < 4; ++e) {
          const float lo = u2f(w[e] << 16), hi = u2f(w[e] & 0xFFFF0000u);
          sm = sm + lo;
          sq = sq + lo * lo;
          sm = sm + hi;
          sq = sq + hi * hi;
        }
      }
      const float mean = sm / (float)a.n;
      const float var = sq / (float)a.n - mean * mean;
      lnst[2 * tid] = mean;
      lnst[2 * tid + 1] = 1.0f / __builtin_sqrtf(var + 1e-5f);
    }
    __syncthreads();
#pragma unroll
    for (int it = 0; it < XL; ++it) {
      const int q = tid + it * 1024;
      if (XQ % 1024 == 0 || q < XQ) {
        const int row = q / (D / 8), c8 = q % (D / 8);
        u32x4* px = reinterpret_cast<u32x4*>(&xs[row * XP + 8 * c8]);
        const u32x4 w = *px;
        const float mean = lnst[2 * row], inv_std = lnst[2 * row + 1];
        const float4 wa = *reinterpret_cast<const float4*>(a.ln2_w + 8 * c8);
        const float4 wb = *reinterpret_cast<const float4*>(a.ln2_w + 8 * c8 + 4);
        const float4 ba = *reinterpret_cast<const float4*>(a.ln2_b + 8 * c8);
        const float4 bb = *reinterpret_cast<const float4*>(a.ln2_b + 8 * c8 + 4);
        const float wv[8] = {wa.x, wa.y, wa.z, wa.w, wb.x, wb.y, wb.z, wb.w};
        const float bv[8] = {ba.x, ba.y, ba.z, ba.w, bb.x, bb.y, bb.z, bb.w};
        u32x4 o;
#pragma unroll
        for (int e = 0; e < 4; ++e) {
          const float lo = u2f(w[e] << 16), hi = u2f(w[e] & 0xFFFF0000u);
          const uint32_t ol = f32_to_bf16(((lo - mean) * inv_std) * wv[2 * e] + bv[2 * e]);
          const uint32_t oh = f32_to_bf16(((hi - mean) * inv_std) * wv[2 * e + 1] + bv[2 * e + 1]);
          o[e] = ol | (oh << 16);
        }
        *px = o;
      }
    }
    // the chunk loop's first barrier orders these stores before FF1's reads
  }
  for (int ch = 0; ch < NC; ++ch) {
    __syncthreads();  // the previous chunk's w1s, hs and w2s are no longer read
    store_chunk();
    if (ch + 1 < NC) load_chunk(ch + 1);
    __syncthreads();
    // FF1 on chunk ch: hidden columns ch HC + 16 TN1 wn1 + 16 q + 4 g + v
    if (ff1_wave) {
      floatx4 acc1[TM1][TN1];
#pragma unroll
      for (int p = 0; p < TM1; ++p)
#pragma unroll
        for (int q = 0; q < TN1; ++q) acc1[p][q] = floatx4{0.f, 0.f, 0.f, 0.f};
#pragma unroll
      for (int ks = 0; ks < D / 32; ++ks) {
        bf16x8 af[TN1], bf[TM1];
#pragma unroll
        for (int q = 0; q < TN1; ++q)
          af[q] = __builtin_bit_cast(bf16x8, *reinterpret_cast<const u32x4*>(
                                                 &w1s[(16 * (TN1 * wn1 + q) + j) * XP + 32 * ks + 8 * g]));
#pragma unroll
        for (int p = 0; p < TM1; ++p)
          bf[p] = __builtin_bit_cast(bf16x8, *reinterpret_cast<const u32x4*>(
                                                 &xs[(16 * (TM1 * wm1 + p) + j) * XP + 32 * ks + 8 * g]));
#pragma unroll
        for (int p = 0; p < TM1; ++p)
#pragma unroll
          for (int q = 0; q < TN1; ++q)
            acc1[p][q] = __builtin_amdgcn_mfma_f32_16x16x32_bf16(af[q], bf[p], acc1[p][q], 0, 0, 0);
      }
#pragma unroll
      for (int p = 0; p < TM1; ++p)
#pragma unroll
        for (int q = 0; q < TN1; ++q) {
          const int n = 16 * (TN1 * wn1 + q) + 4 * g;
          uint16_t o[4];
#pragma unroll
          for (int v = 0; v < 4; ++v) o[v] = f32_to_bf16(gelu<MATH_HW>(acc1[p][q][v] + b1s[n + v]));
          *reinterpret_cast<ushort4*>(&hs[(16 * (TM1 * wm1 + p) + j) * HP + n]) =
              make_ushort4(o[0], o[1], o[2], o[3]);
        }
    }
    __syncthreads();
    // FF2's k-steps of chunk ch
#pragma unroll
    for (int ks = 0; ks < HC / 32; ++ks) {
      bf16x8 af[TN2], bf[TM2];
#pragma unroll
      for (int q = 0; q < TN2; ++q)
        af[q] = __builtin_bit_cast(bf16x8, *reinterpret_cast<const u32x4*>(
                                               &w2s[(16 * (TN2 * wn2 + q) + j) * HP + 32 * ks + 8 * g]));
#pragma unroll
      for (int p = 0; p < TM2; ++p)
        bf[p] = __builtin_bit_cast(bf16x8, *reinterpret_cast<const u32x4*>(
                                               &hs[(16 * (TM2 * wm2 + p) + j) * HP + 32 * ks + 8 * g]));
#pragma unroll
      for (int p = 0; p < TM2; ++p)
#pragma unroll
        for (int q = 0; q < TN2; ++q)
          acc2[p][q] = __builtin_amdgcn_mfma_f32_16x16x32_bf16(af[q], bf[p], acc2[p][q], 0, 0, 0);
    }
  }
  // FF2's epilogue: + b2, + residual, fp32 out (and the bf16 copy)
  float* const rows = reinterpret_cast<float*>(smem);
  if constexpr ((LNF & 2) != 0) __syncthreads();  // every wave is past its last reads of hs, w2s
#pragma unroll
  for (int p = 0; p < TM2; ++p) {
    const int rl = 16 * (TM2 * wm2 + p) + j;
    const int m = m_blk + rl;
    if (m >= a.M) continue;
#pragma unroll
    for (int q = 0; q < TN2; ++q) {
      const int n = 16 * (TN2 * wn2 + q) + 4 * g;
      const float4 rv = *reinterpret_cast<const float4*>(a.res + (size_t)m * D + n);
      const float r4[4] = {rv.x, rv.y, rv.z, rv.w};
      float v[4];
#pragma unroll
      for (int e = 0; e < 4; ++e) v[e] = (acc2[p][q][e] + b2s[n + e]) + r4[e];
      *reinterpret_cast<float4*>(a.C + (size_t)m * D + n) = make_float4(v[0], v[1], v[2], v[3]);
      if ((LNF & 2) != 0)
        *reinterpret_cast<float4*>(rows + rl * RS + n) = make_float4(v[0], v[1], v[2], v[3]);
      if (a.C2)
        *reinterpret_cast<ushort4*>(a.C2 + (size_t)m * D + n) =
            make_ushort4(f32_to_bf16(v[0]), f32_to_bf16(v[1]), f32_to_bf16(v[2]), f32_to_bf16(v[3]));
    }
  }
  if constexpr ((LNF & 2) != 0) {
    __syncthreads();
    // the next layer's LN1: half-wave hw takes rows hw, hw + 32, ...; lane l
    // sums elements l, l + 32, ... in order, then the shuffle-down tree, and
    // lane 0's totals are broadcast; the normalised rows overwrite the LDS rows
    const int hw = tid >> 5, l = tid & 31;
#pragma unroll 1
    for (int rl = hw; rl < BM; rl += 32) {
      float* row = rows + rl * RS;
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
      sm = __shfl(sm, 0, 32);
      sq = __shfl(sq, 0, 32);
      const float mean = sm / (float)a.n;
      const float var = sq / (float)a.n - mean * mean;
      const float inv_std = 1.0f / __builtin_sqrtf(var + 1e-5f);
#pragma unroll
      for (int e = 0; e < D / 32; ++e) {
        const int idx = l + 32 * e;
        row[idx] = ((row[idx] - mean) * inv_std) * a.ln1_w[idx] + a.ln1_b[idx];
      }
    }
    __syncthreads();
    // bf16 xn, eight features (16 bytes) per store
#pragma unroll
    for (int it = 0; it < XL; ++it) {
      const int q = tid + it * 1024;
      if (XQ % 1024 == 0 || q < XQ) {
        const int rl = q / (D / 8), c8 = q % (D / 8);
        const int m = m_blk + rl;
        if (m < a.M) {
          const float* v = rows + rl * RS + 8 * c8;
          u32x4 o;
#pragma unroll
          for (int e = 0; e < 4; ++e)
            o[e] = (uint32_t)f32_to_bf16(v[2 * e]) | ((uint32_t)f32_to_bf16(v[2 * e + 1]) << 16);
          *reinterpret_cast<u32x4*>(a.xn + (size_t)m * D + 8 * c8) = o;
        }
      }
    }
  }
}

hipError_t ffn_bf16(const FfnB16Args& args, hipStream_t s) {
  FfnB16Args a = args;
  if (a.n <= 0) a.n = a.D;  // the LayerNorms' width defaults to the row width
  if (a.M <= 0) return hipSuccess;
  const unsigned blocks = (unsigned)((a.M + 127) / 128);
  switch (a.D) {
    case 256: {
      const bool ln2 = a.ln2_w && a.ln2_b, ln1 = a.xn && a.ln1_w && a.ln1_b;
      if ((a.ln2_w || a.ln2_b) && !ln2) return hipErrorInvalidValue;
      if ((a.xn || a.ln1_w || a.ln1_b) && !ln1) return hipErrorInvalidValue;
#define BOA_FFN(F) \
  BOA_LAUNCH((ffn_bf16_kernel<256, 128, 64, 4, 4, 4, 4, F>), dim3(blocks), dim3(1024), 0, s, a)
      if (ln2 && ln1) BOA_FFN(3);
      else if (ln2) BOA_FFN(1);
      else if (ln1) BOA_FFN(2);
      else BOA_FFN(0);
#undef BOA_FFN
      break;
    }
    default: return hipErrorInvalidValue;
  }
  return hipGetLastError();
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
