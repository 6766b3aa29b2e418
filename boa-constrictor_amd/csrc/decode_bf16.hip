// Decode-step kernels of the bf16 precision (one token per lane).
//
// Activations are bf16 in the 32-blocked layout (feature k of lane m at
// ((k/32) ld + m) 32 + k%32, 64 contiguous bytes per lane and block) except
// the residual stream x, which stays fp32 in the k-blocked layout of the
// fp32 step.  Weights are bf16 in the same 32-blocked layout over their
// output rows.  A v_mfma_f32_16x16x32_bf16 operand slot group (8 k) is then
// one 16-byte load, and each load instruction of a wavefront reads 1 KB.
// The GEMM chain, the epilogue and the per-element sequences are those of
// the bf16 compress kernels, so decode logits equal compress logits.
#include "block_device.h"
#include "boa_kernels.h"

namespace boa {

typedef float floatx4 __attribute__((ext_vector_type(4)));
typedef uint32_t u32x4 __attribute__((ext_vector_type(4)));
typedef __bf16 bf16x8 __attribute__((ext_vector_type(8)));

// ------------------------------------------------------------------- GEMM
// Wave tile 16 features x 16 lanes; lane (i, g) loads, per k-step s of 32,
// W[s][n0+i][8g..8g+7] and X[s][m0+i][8g..8g+7]; accumulator v holds feature
// n0 + 4g + v of lane m0 + i.
// The tile's bias values and fp32 residual, loaded before the K loop so
// that their latency hides behind it.
struct B16Pre {
  float b[4], r[4];
};

__device__ __forceinline__ void dec_b16_prefetch(const DecB16Args& a, int n0, int m, int g,
                                                 B16Pre& p) {
  if (m >= a.M || n0 >= a.N) return;
  const int nb = n0 + 4 * g;
#pragma unroll
  for (int e = 0; e < 4; ++e) {
    p.b[e] = a.bias ? a.bias[min(nb + e, a.N - 1)] : 0.0f;
    p.r[e] = (a.out_mode == DEC_OUT_F32 && a.res && nb + e < a.N) ? a.res[dblk(nb + e, m, a.ldr)]
                                                                  : 0.0f;
  }
}

__device__ __forceinline__ void dec_b16_epilogue(const DecB16Args& a, const floatx4 acc, int n0,
                                                 int m, int g, const B16Pre& pre,
                                                 const ushort4* cs_pre = nullptr) {
  if (m >= a.M || n0 >= a.N) return;
  const int nb = n0 + 4 * g;
  float v[4];
#pragma unroll
  for (int e = 0; e < 4; ++e) {
    float r = acc[e] + pre.b[e];
    if (a.act == ACT_GELU) r = gelu<MATH_HW>(r);
    else if (a.act == ACT_RELU) r = fmaxf(0.0f, r);
    v[e] = r;
  }
  if (a.out_mode == DEC_OUT_ROWMAJOR) {  // logits [M][ldc] fp32
    float* C = reinterpret_cast<float*>(a.C) + (size_t)m * a.ldc + nb;
    if (nb + 4 <= a.N) {
      *reinterpret_cast<float4*>(C) = make_float4(v[0], v[1], v[2], v[3]);
    } else {
#pragma unroll
      for (int e = 0; e < 4; ++e)
        if (nb + e < a.N) C[e] = v[e];
    }
    return;
  }
  if (a.out_mode == DEC_OUT_F32) {  // residual stream: fp32 k-blocked, + res
    float* C = reinterpret_cast<float*>(a.C);
#pragma unroll
    for (int e = 0; e < 4; ++e) {
      const int n = nb + e;
      if (n >= a.N) break;
      float r = v[e];
      if (a.res) r = r + pre.r[e];
      v[e] = r;
      C[dblk(n, m, a.ldc)] = r;
    }
    if (a.C2 && nb + 4 <= a.N)
      *reinterpret_cast<ushort4*>(a.C2 + dblk32(nb, m, a.ldc)) =
          make_ushort4(f32_to_bf16(v[0]), f32_to_bf16(v[1]), f32_to_bf16(v[2]), f32_to_bf16(v[3]));
    return;
  }
  // bf16 32-blocked output; in_proj runs the conv step on its x half
  uint16_t o[4];
  if (a.conv_di > 0 && nb < a.conv_di) {  // conv state: four bf16 per channel and lane
    // every load of the four channels (or their prefetched state) before the
    // first state store, so that they are in flight together
    float4 s0[4], wv[4];
    float cb[4];
#pragma unroll
    for (int e = 0; e < 4; ++e) {
      const ushort4* st = reinterpret_cast<const ushort4*>(a.conv_state) + (size_t)(nb + e) * a.ld_state + m;
      if (cs_pre) {
        const ushort4 h = cs_pre[e];
        s0[e] = make_float4(bf16_to_f32(h.x), bf16_to_f32(h.y), bf16_to_f32(h.z), bf16_to_f32(h.w));
      } else {
        s0[e] = state_ld4h(st, a.state_cached);
      }
      wv[e] = reinterpret_cast<const float4*>(a.conv_w)[nb + e];
      cb[e] = a.conv_b[nb + e];
    }
#pragma unroll
    for (int e = 0; e < 4; ++e) {
      const float x0 = bf16r(v[e]);  // the compress pass reads xz in bf16
      ushort4* st = reinterpret_cast<ushort4*>(a.conv_state) + (size_t)(nb + e) * a.ld_state + m;
      o[e] = f32_to_bf16(conv_step_value<MATH_HW>(cb[e], s0[e], x0, wv[e]));
      state_st4h(st, make_float4(s0[e].y, s0[e].z, s0[e].w, x0), a.state_cached);
    }
    *reinterpret_cast<ushort4*>(a.conv_out + dblk32(nb, m, a.ldc)) = make_ushort4(o[0], o[1], o[2], o[3]);
    return;
  }
  const int row = a.conv_di > 0 ? nb - a.conv_di : nb;
  uint16_t* C = reinterpret_cast<uint16_t*>(a.C);
  if (nb + 4 <= a.N) {
    *reinterpret_cast<ushort4*>(C + dblk32(row, m, a.ldc)) =
        make_ushort4(f32_to_bf16(v[0]), f32_to_bf16(v[1]), f32_to_bf16(v[2]), f32_to_bf16(v[3]));
  } else {
#pragma unroll
    for (int e = 0; e < 4; ++e)
      if (nb + e < a.N) C[dblk32(row + e, m, a.ldc)] = f32_to_bf16(v[e]);
  }
}

template <int KS, int PD>
__global__ __launch_bounds__(256) void dec_b16_gemm_kernel(DecB16Args a) {
  constexpr int UQ = 2;                        // k-steps per prefetch group
  constexpr int G = KS / UQ;                   // groups
  constexpr int R = (PD < G ? PD : G - 1) + 1;  // ring size
  static_assert(KS % UQ == 0, "K must be a multiple of 64");
  const int lane = threadIdx.x & 63;
  const int i = lane & 15, g = lane >> 4;
  const int n_tiles = (a.N + 15) / 16;
  const int m_tiles = (a.M + 15) / 16;
  const int wid = blockIdx.x * (blockDim.x >> 6) + (threadIdx.x >> 6);
  if (wid >= n_tiles * m_tiles) return;  // whole waves exit; no barriers below
  const int n0 = (wid % n_tiles) * 16;
  const int m0 = (wid / n_tiles) * 16;
  const u32x4* wp =
      reinterpret_cast<const u32x4*>(a.W) + (size_t)min(n0 + i, a.ldw - 1) * 4 + g;
  const u32x4* xp = reinterpret_cast<const u32x4*>(a.X) + (size_t)min(m0 + i, a.M - 1) * 4 + g;
  const size_t wq = (size_t)a.ldw * 4, xq = (size_t)a.ldx * 4;  // 16-byte units per k-step
  floatx4 acc = floatx4{0.f, 0.f, 0.f, 0.f};
  B16Pre pre;
  dec_b16_prefetch(a, n0, m0 + i, g, pre);
  u32x4 af[R][UQ], bf[R][UQ];
#define BOA_B16_DLOAD(BUF, S0)                            \
  _Pragma("unroll") for (int q = 0; q < UQ; ++q) {        \
    af[BUF][q] = wp[(size_t)((S0) + q) * wq];             \
    bf[BUF][q] = xp[(size_t)((S0) + q) * xq];             \
  }                                                       \
  __builtin_amdgcn_sched_barrier(0);
#pragma unroll
  for (int p = 0; p < R - 1; ++p) { BOA_B16_DLOAD(p, p * UQ) }
#pragma unroll
  for (int gi = 0; gi < G; ++gi) {
    if (gi + R - 1 < G) { BOA_B16_DLOAD((gi + R - 1) % R, (gi + R - 1) * UQ) }
#pragma unroll
    for (int q = 0; q < UQ; ++q)
      acc = __builtin_amdgcn_mfma_f32_16x16x32_bf16(__builtin_bit_cast(bf16x8, af[gi % R][q]),
                                                    __builtin_bit_cast(bf16x8, bf[gi % R][q]), acc,
                                                    0, 0, 0);
    __builtin_amdgcn_sched_barrier(0);
  }
#undef BOA_B16_DLOAD
  dec_b16_epilogue(a, acc, n0, m0 + i, g, pre);
}

// Register-blocked form for many lanes: a wave runs TM x TN tiles (16 TM
// lanes x 16 TN features), so each operand fragment it loads feeds TN (or
// TM) MFMAs; the k-steps of every tile run in the order of
// dec_b16_gemm_kernel (the same bits).  Loads run two k-steps ahead.
// CONV (in_proj): the conv state of the wave's tiles is loaded with the
// first operands, so that its latency hides behind the K loop (C3 decode
// GEMMs 841 -> 811 us per step; a deeper operand ring, 4 k-steps ahead,
// measured the same, 2 x 4 tiles per wave slower).  The other GEMMs keep
// the registers it takes.
template <int KS, int TM, int TN, bool CONV>
__global__ __launch_bounds__(256) void dec_b16_gemm_blk_kernel(DecB16Args a) {
  constexpr int R = (2 < KS ? 2 : KS - 1) + 1;  // ring size
  const int lane = threadIdx.x & 63;
  const int i = lane & 15, g = lane >> 4;
  const int n_tiles = (a.N + 16 * TN - 1) / (16 * TN);
  const int m_tiles = (a.M + 16 * TM - 1) / (16 * TM);
  const int wid = blockIdx.x * (blockDim.x >> 6) + (threadIdx.x >> 6);
  if (wid >= n_tiles * m_tiles) return;  // whole waves exit; no barriers below
  const int n0 = (wid % n_tiles) * 16 * TN;
  const int m0 = (wid / n_tiles) * 16 * TM;
  const u32x4* wp[TN];
  const u32x4* xp[TM];
#pragma unroll
  for (int t = 0; t < TN; ++t)
    wp[t] = reinterpret_cast<const u32x4*>(a.W) + (size_t)min(n0 + 16 * t + i, a.ldw - 1) * 4 + g;
#pragma unroll
  for (int t = 0; t < TM; ++t)
    xp[t] = reinterpret_cast<const u32x4*>(a.X) + (size_t)min(m0 + 16 * t + i, a.M - 1) * 4 + g;
  const size_t wq = (size_t)a.ldw * 4, xq = (size_t)a.ldx * 4;  // 16-byte units per k-step
  floatx4 acc[TM][TN];
#pragma unroll
  for (int tm = 0; tm < TM; ++tm)
#pragma unroll
    for (int tn = 0; tn < TN; ++tn) acc[tm][tn] = floatx4{0.f, 0.f, 0.f, 0.f};
  u32x4 af[R][TN], bf[R][TM];
#define BOA_B16_BLOAD(BUF, S0)                                                      \
  _Pragma("unroll") for (int t = 0; t < TN; ++t) af[BUF][t] = wp[t][(size_t)(S0) * wq]; \
  _Pragma("unroll") for (int t = 0; t < TM; ++t) bf[BUF][t] = xp[t][(size_t)(S0) * xq]; \
  __builtin_amdgcn_sched_barrier(0);
#pragma unroll
  for (int p = 0; p < R - 1; ++p) { BOA_B16_BLOAD(p, p) }
  // in_proj's conv state of the wave's tiles, loaded with the first
  // operands so that its latency hides behind the K loop
  ushort4 csp[TM][TN][4];
  const bool conv_w = CONV && n0 < a.conv_di;
  if (conv_w) {
#pragma unroll
    for (int tm = 0; tm < TM; ++tm)
#pragma unroll
      for (int tn = 0; tn < TN; ++tn) {
        const int mm = min(m0 + 16 * tm + i, a.M - 1);
        const int nb = n0 + 16 * tn + 4 * g;
#pragma unroll
        for (int e = 0; e < 4; ++e) {
          const ushort4* st = reinterpret_cast<const ushort4*>(a.conv_state) + (size_t)(nb + e) * a.ld_state + mm;
          if (a.state_cached) {
            csp[tm][tn][e] = *st;
          } else {
            const stream_h4 h = __builtin_nontemporal_load(reinterpret_cast<const stream_h4*>(st));
            csp[tm][tn][e] = make_ushort4(h[0], h[1], h[2], h[3]);
          }
        }
      }
  }
#pragma unroll
  for (int st = 0; st < KS; ++st) {
    if (st + R - 1 < KS) { BOA_B16_BLOAD((st + R - 1) % R, st + R - 1) }
#pragma unroll
    for (int tm = 0; tm < TM; ++tm)
#pragma unroll
      for (int tn = 0; tn < TN; ++tn)
        acc[tm][tn] = __builtin_amdgcn_mfma_f32_16x16x32_bf16(
            __builtin_bit_cast(bf16x8, af[st % R][tn]), __builtin_bit_cast(bf16x8, bf[st % R][tm]),
            acc[tm][tn], 0, 0, 0);
    __builtin_amdgcn_sched_barrier(0);
  }
#undef BOA_B16_BLOAD
#pragma unroll
  for (int tm = 0; tm < TM; ++tm)
#pragma unroll
    for (int tn = 0; tn < TN; ++tn) {
      B16Pre pre;
      dec_b16_prefetch(a, n0 + 16 * tn, m0 + 16 * tm + i, g, pre);
      dec_b16_epilogue(a, acc[tm][tn], n0 + 16 * tn, m0 + 16 * tm + i, g, pre,
                       conv_w ? csp[tm][tn] : nullptr);
    }
}

// Workgroup-tiled form for many lanes: a block of four waves owns 64 lanes
// x 64 features.  Per group of KG 32-k steps it copies the lanes' and the
// weight rows' k-blocks (each one contiguous 4 KB span of the 32-blocked
// layouts) into LDS, double-buffered, and wave w runs the 2 x 2 tiles of
// lanes 32 (w / 2) .. + 31 and features 32 (w % 2) .. + 31 from there, the
// k-steps of every tile in the order of dec_b16_gemm_kernel (the same
// bits).  Each operand byte fetched from L2 feeds eight times the MFMAs of
// the wave-per-tile form.
template <int KS, int KG>
__global__ __launch_bounds__(256) void dec_b16_gemm_lds_kernel(DecB16Args a) {
  static_assert(KS % KG == 0, "k-steps must divide into groups");
  constexpr int NG = KS / KG;
  __shared__ __align__(16) u32x4 xs[2][KG][256];  // [buffer][k-step][row * 4 + quarter]
  __shared__ __align__(16) u32x4 ws[2][KG][256];
  const int tid = threadIdx.x, lane = tid & 63, wv = tid >> 6;
  const int i = lane & 15, g = lane >> 4;
  const int n_blocks = (a.N + 63) / 64;
  const int m0 = (blockIdx.x / n_blocks) * 64, n0 = (blockIdx.x % n_blocks) * 64;
  // staging: thread t copies quarter t % 4 of row t / 4 of each k-block
  const int sr = tid >> 2, sq = tid & 3;
  const int ms = min(m0 + sr, a.M - 1), ns = min(n0 + sr, a.ldw - 1);
  const u32x4* X4 = reinterpret_cast<const u32x4*>(a.X);
  const u32x4* W4 = reinterpret_cast<const u32x4*>(a.W);
  u32x4 xr[KG], wr[KG];
#define BOA_B16_GLOAD(S0)                                                         \
  _Pragma("unroll") for (int kg = 0; kg < KG; ++kg) {                             \
    xr[kg] = X4[((size_t)((S0) + kg) * a.ldx + ms) * 4 + sq];                     \
    wr[kg] = W4[((size_t)((S0) + kg) * a.ldw + ns) * 4 + sq];                     \
  }
#define BOA_B16_GSTORE(BUF)                                                       \
  _Pragma("unroll") for (int kg = 0; kg < KG; ++kg) {                             \
    xs[BUF][kg][tid] = xr[kg];                                                    \
    ws[BUF][kg][tid] = wr[kg];                                                    \
  }
  const int lr = 32 * (wv >> 1), fr = 32 * (wv & 1);
  floatx4 acc[2][2];
#pragma unroll
  for (int tm = 0; tm < 2; ++tm)
#pragma unroll
    for (int tn = 0; tn < 2; ++tn) acc[tm][tn] = floatx4{0.f, 0.f, 0.f, 0.f};
  // in_proj's conv state of the wave's four tiles, loaded before the K loop
  // (with the grouped epilogue loads: C5 probe decode 0.992 -> 1.082 MB/s,
  // C3 4.60 -> 4.73)
  ushort4 csp[2][2][4];
  const bool conv_blk = a.conv_di > 0 && n0 < a.conv_di;
  if (conv_blk) {
#pragma unroll
    for (int tm = 0; tm < 2; ++tm)
#pragma unroll
      for (int tn = 0; tn < 2; ++tn) {
        const int mm = min(m0 + lr + 16 * tm + i, a.M - 1);
        const int nb = n0 + fr + 16 * tn + 4 * g;
#pragma unroll
        for (int e = 0; e < 4; ++e) {
          const ushort4* st = reinterpret_cast<const ushort4*>(a.conv_state) + (size_t)(nb + e) * a.ld_state + mm;
          if (a.state_cached) {
            csp[tm][tn][e] = *st;
          } else {
            const stream_h4 h = __builtin_nontemporal_load(reinterpret_cast<const stream_h4*>(st));
            csp[tm][tn][e] = make_ushort4(h[0], h[1], h[2], h[3]);
          }
        }
      }
  }
  BOA_B16_GLOAD(0)
  BOA_B16_GSTORE(0)
  __syncthreads();
  for (int gi = 0; gi < NG; ++gi) {
    const int cur = gi & 1;
    if (gi + 1 < NG) { BOA_B16_GLOAD((gi + 1) * KG) }
#pragma unroll
    for (int kg = 0; kg < KG; ++kg) {
      u32x4 bf[2], af[2];
#pragma unroll
      for (int t = 0; t < 2; ++t) {
        bf[t] = xs[cur][kg][(lr + 16 * t + i) * 4 + g];
        af[t] = ws[cur][kg][(fr + 16 * t + i) * 4 + g];
      }
#pragma unroll
      for (int tm = 0; tm < 2; ++tm)
#pragma unroll
        for (int tn = 0; tn < 2; ++tn)
          acc[tm][tn] = __builtin_amdgcn_mfma_f32_16x16x32_bf16(
              __builtin_bit_cast(bf16x8, af[tn]), __builtin_bit_cast(bf16x8, bf[tm]), acc[tm][tn],
              0, 0, 0);
    }
    if (gi + 1 < NG) { BOA_B16_GSTORE(cur ^ 1) }
    __syncthreads();
  }
#undef BOA_B16_GLOAD
#undef BOA_B16_GSTORE
#pragma unroll
  for (int tm = 0; tm < 2; ++tm)
#pragma unroll
    for (int tn = 0; tn < 2; ++tn) {
      B16Pre pre;
      dec_b16_prefetch(a, n0 + fr + 16 * tn, m0 + lr + 16 * tm + i, g, pre);
      dec_b16_epilogue(a, acc[tm][tn], n0 + fr + 16 * tn, m0 + lr + 16 * tm + i, g, pre,
                       conv_blk ? csp[tm][tn] : nullptr);
    }
}

// Block-tiled form for many lanes and outputs 512 wide or more: a block of
// four waves owns 128 lanes x 128 features, wave w the 4 x 4 tiles of lanes
// 64 (w / 2) .. + 63 and features 64 (w % 2) .. + 63.  The
// operands go straight from global memory to LDS (global_load_lds, 16 bytes
// a lane), one 32-k step a stage, three stages in flight in a ring of four,
// so each operand byte passes the vector memory path once per block tile
// (the register-blocked form re-read each fragment per 32 x 32 tile, which
// kept its texture-address units busy half its time; the 64 x 64 LDS form
// stages through registers one group ahead, which its MFMAs cannot cover).
// A stage's tile of one operand holds row r's 16-byte quarter q at position
// q ^ ((r >> 2) & 3), so that the 16 lanes of a ds_read_b128 pass read 16
// distinct bank groups.  The stage's reads and barrier bypass the
// compiler's waits (lds_read128, lds_barrier: its own would wait for every
// copy in flight).  Blocks map to XCDs by t128_block.  Every tile's k-steps
// run in the order of dec_b16_gemm_kernel (the same bits).  The epilogue
// (dec_b16_epilogue's, for bf16 or fp32 + residual outputs) walks the tiles
// a feature column at a time, loading the column's bias (and in_proj's conv
// taps) once; in_proj loads column tn + 1's conv state while column tn is
// computed.
constexpr int T128_RING = 4;  // LDS stages; T128_RING - 1 in flight

// in_proj's conv blocks: per feature column tn of the wave (features nw +
// 16 tn + 4 g + e), the conv state of its tiles' lanes and the column's bias,
// taps and conv biases, loaded one column ahead (the column being computed
// waits only for its own loads).  SC: the state's cache policy (1 cached, 0
// streamed) at compile time; a runtime choice joins two loads in a register
// copy that the compiler guards with a wait for every load in flight.
template <int TMW, int SC>
__device__ __forceinline__ void t128_conv_epilogue(const DecB16Args& a, const floatx4 (&acc)[TMW][4],
                                                   int nw, int mw, int g) {
  struct ColOps {
    ushort4 cs[TMW][4];
    float4 bias, cw[4], cb;
  };
  ColOps col[2];
  auto load_col = [&](int tn, ColOps& o) {
    const int nb = nw + 16 * tn + 4 * g;  // < conv_di <= N: in bounds
#pragma unroll
    for (int tm = 0; tm < TMW; ++tm) {
      const int mm = min(mw + 16 * tm, a.M - 1);
#pragma unroll
      for (int e = 0; e < 4; ++e) {
        const ushort4* sp = reinterpret_cast<const ushort4*>(a.conv_state) + (size_t)(nb + e) * a.ld_state + mm;
        if constexpr (SC) {
          o.cs[tm][e] = *sp;
        } else {
          const stream_h4 h = __builtin_nontemporal_load(reinterpret_cast<const stream_h4*>(sp));
          o.cs[tm][e] = make_ushort4(h[0], h[1], h[2], h[3]);
        }
      }
    }
    o.bias = *reinterpret_cast<const float4*>(a.bias + nb);
#pragma unroll
    for (int e = 0; e < 4; ++e) o.cw[e] = reinterpret_cast<const float4*>(a.conv_w)[nb + e];
    o.cb = *reinterpret_cast<const float4*>(a.conv_b + nb);
  };
  load_col(0, col[0]);
#pragma unroll
  for (int tn = 0; tn < 4; ++tn) {
    if (tn + 1 < 4) load_col(tn + 1, col[(tn + 1) & 1]);
    const ColOps& c = col[tn & 1];
    const int nb = nw + 16 * tn + 4 * g;
    const float bb[4] = {c.bias.x, c.bias.y, c.bias.z, c.bias.w};
    const float cbb[4] = {c.cb.x, c.cb.y, c.cb.z, c.cb.w};
    // every use of a loaded value is unconditional; only the stores test
    // m < M (a use under the test would be waited for again, with every
    // load and store in flight, after each tile row)
#pragma unroll
    for (int tm = 0; tm < TMW; ++tm) {
      const int m = mw + 16 * tm;
      uint16_t o[4];
      float4 ns[4];
#pragma unroll
      for (int e = 0; e < 4; ++e) {
        float r = acc[tm][tn][e] + bb[e];
        if (a.act == ACT_GELU) r = gelu<MATH_HW>(r);
        else if (a.act == ACT_RELU) r = fmaxf(0.0f, r);
        const ushort4 h = c.cs[tm][e];
        const float4 s0 = make_float4(bf16_to_f32(h.x), bf16_to_f32(h.y), bf16_to_f32(h.z),
                                      bf16_to_f32(h.w));
        const float x0 = bf16r(r);  // the compress pass reads xz in bf16
        o[e] = f32_to_bf16(conv_step_value<MATH_HW>(cbb[e], s0, x0, c.cw[e]));
        ns[e] = make_float4(s0.y, s0.z, s0.w, x0);
      }
      if (m < a.M) {
#pragma unroll
        for (int e = 0; e < 4; ++e)
          state_st4h(reinterpret_cast<ushort4*>(a.conv_state) + (size_t)(nb + e) * a.ld_state + m,
                     ns[e], SC != 0);
        *reinterpret_cast<ushort4*>(a.conv_out + dblk32(nb, m, a.ldc)) =
            make_ushort4(o[0], o[1], o[2], o[3]);
      }
    }
    __builtin_amdgcn_sched_barrier(0);
  }
}

// SC: in_proj's conv state cache policy (t128_conv_epilogue; 0 otherwise).
// BM x BN blocks (128 x 128, or 64 x 64 for the 256-wide outputs), four
// waves of (BM / 2) x (BN / 2).
template <int KS, bool CONV, bool F32, int SC, int BM = 128, int BN = 128>
__global__ __launch_bounds__(256) __attribute__((amdgpu_waves_per_eu(2, 2)))
void dec_b16_gemm_t128_kernel(DecB16Args a) {
  static_assert(!CONV || BN == 128, "the conv epilogue walks 64-feature wave columns");
  constexpr int NR = T128_RING, PF = (NR - 1 < KS ? NR - 1 : KS);  // stages issued ahead
  constexpr int TMW = BM / 32, TNW = BN / 32;  // lane and feature tiles per wave
  constexpr int NQ = (BM + BN) / 16;           // 1 KB copies per stage
  constexpr int IPW = NQ / 4;                  // of them per wave
  // [ring stage][X rows 0 .. BM-1, then W rows 0 .. BN-1][row * 4 + quarter]
  __shared__ __align__(16) u32x4 sm[NR][(BM + BN) * 4];
  const int tid = threadIdx.x, lane = tid & 63, wv = tid >> 6;
  const int i = lane & 15, g = lane >> 4;
  const int2 mn = t128_block(blockIdx.x, (a.M + BM - 1) / BM, (a.N + BN - 1) / BN);
  const int m0 = mn.x * BM, n0 = mn.y * BN;
  const u32x4* X4 = reinterpret_cast<const u32x4*>(a.X);
  const u32x4* W4 = reinterpret_cast<const u32x4*>(a.W);
  // DMA of k-step st: wave wv issues copies IPW wv .. IPW wv + IPW - 1 of
  // the stage's NQ (the first BM / 16 fill X, the rest W); lane L of copy j
  // of an operand fills position 64 j + L: row (64 j + L) / 4, quarter L % 4
  auto issue = [&](int st) {
    const int buf = st % NR;
#pragma unroll
    for (int u = 0; u < IPW; ++u) {
      const int q = IPW * wv + u;
      const bool xop = q < BM / 16;
      const int j = xop ? q : q - BM / 16;
      const int pos = 64 * j + lane, row = pos >> 2, qd = pos & 3;
      const int gq = qd ^ ((row >> 2) & 3);
      const u32x4* src = xop ? X4 + ((size_t)st * a.ldx + min(m0 + row, a.M - 1)) * 4 + gq
                             : W4 + ((size_t)st * a.ldw + min(n0 + row, a.ldw - 1)) * 4 + gq;
      __builtin_amdgcn_global_load_lds(
          (const void*)src,
          (__attribute__((address_space(3))) void*)(&sm[buf][(xop ? 0 : BM * 4) + 64 * j]), 16, 0,
          0);
    }
  };
  const int wm = wv >> 1, wn = wv & 1;
  floatx4 acc[TMW][TNW];
#pragma unroll
  for (int tm = 0; tm < TMW; ++tm)
#pragma unroll
    for (int tn = 0; tn < TNW; ++tn) acc[tm][tn] = floatx4{0.f, 0.f, 0.f, 0.f};
#pragma unroll
  for (int st = 0; st < PF; ++st) issue(st);
#pragma unroll 1
  for (int st = 0; st < KS; ++st) {
    // this wave's copies of stage st have landed (the younger in-flight
    // stages, IPW copies each, may still run); after the barrier every
    // wave's have, and every wave is done with stage st - 1's buffer
    vm_wait(IPW * min(PF - 1, KS - 1 - st));
    lds_barrier();
    if (st + PF < KS) issue(st + PF);
    const int buf = st % NR;
    u32x4 xf[4], wf[4];
#pragma unroll
    for (int t = 0; t < 4; ++t) {
      if (t < TMW) {
        const int rx = (BM / 2) * wm + 16 * t + i;
        xf[t] = lds_read128(&sm[buf][rx * 4 + (g ^ ((rx >> 2) & 3))]);
      }
      if (t < TNW) {
        const int rw = (BN / 2) * wn + 16 * t + i;
        wf[t] = lds_read128(&sm[buf][BM * 4 + rw * 4 + (g ^ ((rw >> 2) & 3))]);
      }
    }
    if constexpr (TMW == 4 && TNW == 4) lds_wait8(xf[0], xf[1], xf[2], xf[3], wf[0], wf[1], wf[2], wf[3]);
    else lds_wait4(xf[0], xf[1], wf[0], wf[1]);
#pragma unroll
    for (int tm = 0; tm < TMW; ++tm)
#pragma unroll
      for (int tn = 0; tn < TNW; ++tn)
        acc[tm][tn] = __builtin_amdgcn_mfma_f32_16x16x32_bf16(
            __builtin_bit_cast(bf16x8, wf[tn]), __builtin_bit_cast(bf16x8, xf[tm]), acc[tm][tn], 0,
            0, 0);
  }
  // epilogue: bias and activation; bf16 outputs (in_proj's x half runs the
  // conv step) or fp32 + residual (and the bf16 copy), as dec_b16_epilogue
  if constexpr (CONV) {
    if (n0 < a.conv_di) {
      t128_conv_epilogue<TMW, SC>(a, acc, n0 + 64 * wn, m0 + (BM / 2) * wm + i, g);
      return;
    }
  }
  // column tn + 1's bias (and residual, fp32 outputs) load while column tn
  // is computed; the loaded values are used unconditionally and only the
  // stores test m < M (as in t128_conv_epilogue)
  struct ColOps {
    float4 bias;
    float res[F32 ? TMW : 1][4];
  };
  ColOps col[2];
  auto load_col = [&](int tn, ColOps& o) {
    const int nb = min(n0 + (BN / 2) * wn + 16 * tn + 4 * g, a.N - 4);  // N % 4 == 0
    o.bias = a.bias ? *reinterpret_cast<const float4*>(a.bias + nb) : make_float4(0.f, 0.f, 0.f, 0.f);
    if constexpr (F32) {
      if (a.res) {
#pragma unroll
        for (int tm = 0; tm < TMW; ++tm) {
          const int mc = min(m0 + (BM / 2) * wm + 16 * tm + i, a.M - 1);
#pragma unroll
          for (int e = 0; e < 4; ++e) o.res[tm][e] = a.res[dblk(nb + e, mc, a.ldr)];
        }
      }
    }
  };
  load_col(0, col[0]);
#pragma unroll
  for (int tn = 0; tn < TNW; ++tn) {
    if (tn + 1 < TNW) load_col(tn + 1, col[(tn + 1) & 1]);
    const ColOps& c = col[tn & 1];
    const int nb = n0 + (BN / 2) * wn + 16 * tn + 4 * g;
    const float bb[4] = {c.bias.x, c.bias.y, c.bias.z, c.bias.w};
#pragma unroll
    for (int tm = 0; tm < TMW; ++tm) {
      const int m = m0 + (BM / 2) * wm + 16 * tm + i;
      float v[4];
#pragma unroll
      for (int e = 0; e < 4; ++e) {
        float r = acc[tm][tn][e] + bb[e];
        if (a.act == ACT_GELU) r = gelu<MATH_HW>(r);
        else if (a.act == ACT_RELU) r = fmaxf(0.0f, r);
        v[e] = r;
      }
      if constexpr (F32) {  // residual stream: fp32 k-blocked, + res
        if (a.res) {
#pragma unroll
          for (int e = 0; e < 4; ++e) v[e] = v[e] + c.res[tm][e];
        }
        if (m < a.M && nb < a.N) {
          float* C = reinterpret_cast<float*>(a.C);
#pragma unroll
          for (int e = 0; e < 4; ++e) C[dblk(nb + e, m, a.ldc)] = v[e];
          if (a.C2)
            *reinterpret_cast<ushort4*>(a.C2 + dblk32(nb, m, a.ldc)) =
                make_ushort4(f32_to_bf16(v[0]), f32_to_bf16(v[1]), f32_to_bf16(v[2]), f32_to_bf16(v[3]));
        }
      } else if (m < a.M && nb < a.N) {
        uint16_t* C = reinterpret_cast<uint16_t*>(a.C);
        const int row = a.conv_di > 0 ? nb - a.conv_di : nb;
        *reinterpret_cast<ushort4*>(C + dblk32(row, m, a.ldc)) =
            make_ushort4(f32_to_bf16(v[0]), f32_to_bf16(v[1]), f32_to_bf16(v[2]), f32_to_bf16(v[3]));
      }
    }
    __builtin_amdgcn_sched_barrier(0);
  }
}

namespace {
hipError_t dec_b16_lds_launch(const DecB16Args& a, hipStream_t s) {
  const dim3 grid(((a.M + 63) / 64) * ((a.N + 63) / 64)), block(256);
  switch (a.K) {
    case 64: BOA_LAUNCH((dec_b16_gemm_lds_kernel<2, 2>), grid, block, 0, s, a); break;
    case 128: BOA_LAUNCH((dec_b16_gemm_lds_kernel<4, 4>), grid, block, 0, s, a); break;
    case 256: BOA_LAUNCH((dec_b16_gemm_lds_kernel<8, 4>), grid, block, 0, s, a); break;
    case 512: BOA_LAUNCH((dec_b16_gemm_lds_kernel<16, 4>), grid, block, 0, s, a); break;
    case 1024: BOA_LAUNCH((dec_b16_gemm_lds_kernel<32, 4>), grid, block, 0, s, a); break;
    case 2048: BOA_LAUNCH((dec_b16_gemm_lds_kernel<64, 4>), grid, block, 0, s, a); break;
    default: return hipErrorInvalidValue;
  }
  return hipGetLastError();
}

template <bool CONV, bool F32, int SC = 0, int BM = 128, int BN = 128>
hipError_t dec_b16_t128_launch(const DecB16Args& a, hipStream_t s) {
  const dim3 grid(((a.M + BM - 1) / BM) * ((a.N + BN - 1) / BN)), block(256);
#define BOA_T128(KSv) BOA_LAUNCH((dec_b16_gemm_t128_kernel<KSv, CONV, F32, SC, BM, BN>), grid, block, 0, s, a)
  switch (a.K) {
    case 64: BOA_T128(2); break;
    case 128: BOA_T128(4); break;
    case 256: BOA_T128(8); break;
    case 512: BOA_T128(16); break;
    case 1024: BOA_T128(32); break;
    case 2048: BOA_T128(64); break;
    default: return hipErrorInvalidValue;
  }
#undef BOA_T128
  return hipGetLastError();
}

template <int TM, int TN, bool CONV>
hipError_t dec_b16_blk_launch(const DecB16Args& a, hipStream_t s) {
  const int tiles = ((a.N + 16 * TN - 1) / (16 * TN)) * ((a.M + 16 * TM - 1) / (16 * TM));
  const dim3 grid((tiles + 3) / 4), block(256);
  switch (a.K) {
    case 64: BOA_LAUNCH((dec_b16_gemm_blk_kernel<2, TM, TN, CONV>), grid, block, 0, s, a); break;
    case 128: BOA_LAUNCH((dec_b16_gemm_blk_kernel<4, TM, TN, CONV>), grid, block, 0, s, a); break;
    case 256: BOA_LAUNCH((dec_b16_gemm_blk_kernel<8, TM, TN, CONV>), grid, block, 0, s, a); break;
    case 512: BOA_LAUNCH((dec_b16_gemm_blk_kernel<16, TM, TN, CONV>), grid, block, 0, s, a); break;
    case 1024: BOA_LAUNCH((dec_b16_gemm_blk_kernel<32, TM, TN, CONV>), grid, block, 0, s, a); break;
    case 2048: BOA_LAUNCH((dec_b16_gemm_blk_kernel<64, TM, TN, CONV>), grid, block, 0, s, a); break;
    default: return hipErrorInvalidValue;
  }
  return hipGetLastError();
}
}  // namespace

hipError_t dec_b16_gemm(const DecB16Args& a, hipStream_t s) {
  if (a.M <= 0 || a.N <= 0) return hipSuccess;
  if (a.ldw < (a.N + 15) / 16 * 16 || a.ldx < a.M || (a.conv_di % 16) ||
      (a.out_mode != DEC_OUT_ROWMAJOR && a.ldc < a.M) || (a.res && a.ldr < a.M))
    return hipErrorInvalidValue;
  // From 2048 lanes on:
  // - outputs 512 wide or more (in_proj and FF1; at d_model 512 also
  //   out_proj and FF2): the 128 x 128 blocks (C3 decode GEMMs 809 -> 716
  //   us per step, decompress 4.88 -> 5.15 MB/s; C5 probe 5.58 -> 4.73 ms,
  //   1.05 -> 1.11 MB/s, then out_proj and FF2 4.24 -> 3.84 ms, 1.153 ->
  //   1.187 MB/s; 64-lane blocks for the 256-wide out_proj and FF2 of C3
  //   were slower, 708 -> 774 us), in 64 x 128 blocks where 128 x 128 ones
  //   would leave under two per CU (C5's 512-wide out_proj, FF2 and head.1
  //   at 8192 lanes: decode GEMMs 2174 -> 2108 us per step; the same for
  //   its 2048-wide FF1, 1024 blocks, was slower);
  // - outputs under 512 wide with K >= 512 (C3's FF2, fp32 + residual; its
  //   out_proj and x_proj, bf16; C5's x_proj), and bf16 ones with K = 256
  //   (C3's head.1): the same form in 64 x 64 blocks (C3 probe decode GEMMs
  //   644 -> 635 us per step for FF2, then 632 -> 616 with out_proj and
  //   x_proj, 626 -> 619 with head.1, against the 64 x 64 register-staged
  //   and the 2 x 2-tile blocks; two to eight waves per SIMD measured even);
  //   x_proj's 48 or 96 columns fill the last block in part (the weight
  //   rows past N read the last row, the stores test n < N);
  // - the other GEMMs: 2 x 2 tiles per wave for K <= 256 (C3 decode 3.76 ->
  //   4.40 MB/s against one tile per wave; 4 x 4, 2 x 1 and 1 x 2 were
  //   slower) and the 64 x 64 LDS-tiled blocks for K >= 512 (4.40 -> 4.54
  //   MB/s at C3, 0.95 -> 0.98 at C5)
  if (a.M >= 2048) {
    if ((a.out_mode == DEC_OUT_B16 || a.out_mode == DEC_OUT_F32) && a.N >= 512 &&
        a.conv_di % 128 == 0 && (a.conv_di == 0 || a.bias)) {
      // fewer than two 128 x 128 blocks per CU: 64 x 128 blocks
      const int cus = a.n_cus > 0 ? a.n_cus : 256;
      const bool rows64 = (int64_t)((a.M + 127) / 128) * ((a.N + 127) / 128) < 2 * (int64_t)cus;
      if (a.out_mode == DEC_OUT_F32)
        return rows64 ? dec_b16_t128_launch<false, true, 0, 64, 128>(a, s)
                      : dec_b16_t128_launch<false, true>(a, s);
      if (a.conv_di == 0)
        return rows64 ? dec_b16_t128_launch<false, false, 0, 64, 128>(a, s)
                      : dec_b16_t128_launch<false, false>(a, s);
      return a.state_cached ? dec_b16_t128_launch<true, false, 1>(a, s)
                            : dec_b16_t128_launch<true, false, 0>(a, s);
    }
    if (a.out_mode == DEC_OUT_F32 && a.N % 64 == 0 && a.K >= 512)
      return dec_b16_t128_launch<false, true, 0, 64, 64>(a, s);
    if (a.out_mode == DEC_OUT_B16 && a.conv_di == 0 && a.N % 16 == 0 && a.K >= 256)
      return dec_b16_t128_launch<false, false, 0, 64, 64>(a, s);
    if (a.K >= 512) return dec_b16_lds_launch(a, s);
    return a.conv_di > 0 ? dec_b16_blk_launch<2, 2, true>(a, s) : dec_b16_blk_launch<2, 2, false>(a, s);
  }
  const int tiles = ((a.N + 15) / 16) * ((a.M + 15) / 16);
  const dim3 grid((tiles + 3) / 4), block(256);
  switch (a.K) {
    case 64: BOA_LAUNCH((dec_b16_gemm_kernel<2, 2>), grid, block, 0, s, a); break;
    case 128: BOA_LAUNCH((dec_b16_gemm_kernel<4, 2>), grid, block, 0, s, a); break;
    case 256: BOA_LAUNCH((dec_b16_gemm_kernel<8, 2>), grid, block, 0, s, a); break;
    case 512: BOA_LAUNCH((dec_b16_gemm_kernel<16, 2>), grid, block, 0, s, a); break;
    case 1024: BOA_LAUNCH((dec_b16_gemm_kernel<32, 2>), grid, block, 0, s, a); break;
    case 2048: BOA_LAUNCH((dec_b16_gemm_kernel<64, 2>), grid, block, 0, s, a); break;
    default: return hipErrorInvalidValue;
  }
  return hipGetLastError();
}

// Weight relayout: W [K][ldw_in] fp32 (the fp32 compress layout) -> bf16
// 32-blocked over its output columns [K/32][ldn][32]; logical column j maps
// to source column j (j < zs), a zero column (zs <= j < ze) or source column
// j - (ze - zs) (j >= ze).
__global__ void dec_b16_weight_kernel(const float* __restrict__ w, int ldw_in, int n_src,
                                      uint16_t* out, int K, int ldn, int zs, int ze) {
  const size_t idx = (size_t)blockIdx.x * blockDim.x + threadIdx.x;
  if (idx >= (size_t)K * ldn) return;
  const int k = (int)(idx / ldn), j = (int)(idx % ldn);
  const int n = j < zs ? j : (j < ze ? -1 : j - (ze - zs));
  out[dblk32(k, j, ldn)] = (n >= 0 && n < n_src) ? f32_to_bf16(w[(size_t)k * ldw_in + n]) : 0;
}

hipError_t launch_dec_b16_weight(const float* w, int ldw_in, int n_src, uint16_t* out, int K,
                                 int ldn, int zs, int ze, hipStream_t s) {
  if (K % 32 || ldn % 16 || n_src > ldw_in || zs > ze) return hipErrorInvalidValue;
  const size_t n = (size_t)K * ldn;
  BOA_LAUNCH(dec_b16_weight_kernel, dim3((unsigned)((n + 255) / 256)), dim3(256), 0, s, w,
                     ldw_in, n_src, out, K, ldn, zs, ze);
  return hipGetLastError();
}

// -------------------------------------------------------------- LayerNorm
// As the fp32 step LayerNorm (16 lanes per 256-thread block, reference
// reduction orders), reading fp32 k-blocked x (LN1), the embedding (layer
// 0, which also stores x) or bf16 32-blocked activations (LN2), and writing
// bf16 32-blocked output.
enum { LN_IN_F32 = 0, LN_IN_EMB = 1, LN_IN_B16 = 2 };

template <int MODE, int NB, int IN>
__global__ __launch_bounds__(256) void dec_b16_ln_kernel(const float* __restrict__ emb,
                                                         const uint8_t* __restrict__ tok, float* xt,
                                                         const void* src, uint16_t* xnt,
                                                         const float* __restrict__ w,
                                                         const float* __restrict__ b, int M,
                                                         int ld, int* t_counter, int n) {
  constexpr int d = NB * 16;
  constexpr int S = d + 4;
  __shared__ __align__(16) float tile[16 * S];
  __shared__ float stats[32];
  if (t_counter && blockIdx.x == 0 && threadIdx.x == 0) *t_counter += 1;
  const int t = threadIdx.x;
  const int m0 = blockIdx.x * 16;
  {  // stage the 16 rows in natural feature order
    const int j = (t >> 2) & 15, a4 = t & 3;
    const int m = min(m0 + j, M - 1);
    if (IN == LN_IN_B16) {
      // thread: 8 features (16 bytes) of a 32-feature block
      const uint16_t* s16 = reinterpret_cast<const uint16_t*>(src);
      for (int kb = t >> 6; kb < d / 32; kb += 4) {
        const u32x4 r = *reinterpret_cast<const u32x4*>(s16 + dblk32(32 * kb + 8 * a4, m, ld));
        float* row = tile + j * S + 32 * kb + 8 * a4;
#pragma unroll
        for (int e = 0; e < 4; ++e) {
          row[2 * e] = u2f(r[e] << 16);
          row[2 * e + 1] = u2f(r[e] & 0xFFFF0000u);
        }
      }
    } else {
      const float* erow = IN == LN_IN_EMB ? emb + (size_t)tok[m] * d : nullptr;
      const float* s32 = reinterpret_cast<const float*>(src);
      for (int kb = t >> 6; kb < NB; kb += 4) {
        float* row = tile + j * S + 16 * kb;
        if (IN == LN_IN_EMB) {
          const float4 v = *reinterpret_cast<const float4*>(erow + 16 * kb + 4 * a4);
          row[4 * a4] = v.x; row[4 * a4 + 1] = v.y; row[4 * a4 + 2] = v.z; row[4 * a4 + 3] = v.w;
        } else {
          const float4 v = *reinterpret_cast<const float4*>(s32 + ((size_t)kb * ld + m) * 16 + 4 * a4);
          row[dperm(4 * a4)] = v.x; row[dperm(4 * a4 + 1)] = v.y;
          row[dperm(4 * a4 + 2)] = v.z; row[dperm(4 * a4 + 3)] = v.w;
        }
      }
    }
  }
  __syncthreads();
  if (MODE == 1) {
    const int lj = t >> 4, l = t & 15;
    const float* row = tile + lj * S;
    float s0 = 0.0f, q0 = 0.0f, s1 = 0.0f, q1 = 0.0f;
    for (int k = l; k < d; k += 32) { const float x = row[k]; s0 = s0 + x; q0 = q0 + x * x; }
    for (int k = l + 16; k < d; k += 32) { const float x = row[k]; s1 = s1 + x; q1 = q1 + x * x; }
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
  } else if (t < 16) {
    const float4* row = reinterpret_cast<const float4*>(tile + t * S);
    float sum = 0.0f, sq = 0.0f;
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
  const int j = (t >> 2) & 15, a4 = t & 3;
  if (m0 + j >= M) return;
  const float mean = stats[2 * j], rstd = stats[2 * j + 1];
  const float* row = tile + j * S;
  for (int kb = t >> 6; kb < d / 32; kb += 4) {  // 8 features per thread and block
    const int k0 = 32 * kb + 8 * a4;
    uint32_t r[4];
#pragma unroll
    for (int e = 0; e < 4; ++e) {
      const int k = k0 + 2 * e;
      const float o0 = ((row[k] - mean) * rstd) * w[k] + b[k];
      const float o1 = ((row[k + 1] - mean) * rstd) * w[k + 1] + b[k + 1];
      r[e] = (uint32_t)f32_to_bf16(o0) | ((uint32_t)f32_to_bf16(o1) << 16);
    }
    *reinterpret_cast<u32x4*>(xnt + dblk32(k0, m0 + j, ld)) = u32x4{r[0], r[1], r[2], r[3]};
  }
  if (IN == LN_IN_EMB) {  // x = the embedding row, fp32 k-blocked
    for (int kb = t >> 6; kb < NB; kb += 4) {
      const float* rr = row + 16 * kb;
      *reinterpret_cast<float4*>(xt + ((size_t)kb * ld + m0 + j) * 16 + 4 * a4) =
          make_float4(rr[dperm(4 * a4)], rr[dperm(4 * a4 + 1)], rr[dperm(4 * a4 + 2)],
                      rr[dperm(4 * a4 + 3)]);
    }
  }
}

template <int MODE, int IN>
static hipError_t dec_b16_ln_go(const float* emb, const uint8_t* tok, float* xt, const void* src,
                                uint16_t* xnt, const float* w, const float* b, int M, int d, int n,
                                int ld, int* t_counter, hipStream_t s) {
  const dim3 grid((M + 15) / 16), block(256);
  switch (d) {
    case 64: BOA_LAUNCH((dec_b16_ln_kernel<MODE, 4, IN>), grid, block, 0, s, emb, tok, xt, src, xnt, w, b, M, ld, t_counter, n); break;
    case 128: BOA_LAUNCH((dec_b16_ln_kernel<MODE, 8, IN>), grid, block, 0, s, emb, tok, xt, src, xnt, w, b, M, ld, t_counter, n); break;
    case 256: BOA_LAUNCH((dec_b16_ln_kernel<MODE, 16, IN>), grid, block, 0, s, emb, tok, xt, src, xnt, w, b, M, ld, t_counter, n); break;
    case 512: BOA_LAUNCH((dec_b16_ln_kernel<MODE, 32, IN>), grid, block, 0, s, emb, tok, xt, src, xnt, w, b, M, ld, t_counter, n); break;
    default: return hipErrorInvalidValue;
  }
  return hipGetLastError();
}

// LN1: from the embedding (emb != null; also stores x) or from fp32 x.
hipError_t launch_dec_b16_ln1(const float* emb, const uint8_t* tok, float* xt, uint16_t* xnt,
                              const float* w, const float* b, int M, int d, int n, int ld,
                              int* t_counter, hipStream_t s) {
  return emb ? dec_b16_ln_go<1, LN_IN_EMB>(emb, tok, xt, nullptr, xnt, w, b, M, d, n, ld,
                                           t_counter, s)
             : dec_b16_ln_go<1, LN_IN_F32>(nullptr, nullptr, nullptr, xt, xnt, w, b, M, d, n, ld,
                                           t_counter, s);
}

hipError_t launch_dec_b16_ln2(const uint16_t* src, uint16_t* xnt, const float* w, const float* b,
                              int M, int d, int n, int ld, hipStream_t s) {
  return dec_b16_ln_go<2, LN_IN_B16>(nullptr, nullptr, nullptr, src, xnt, w, b, M, d, n, ld,
                                     nullptr, s);
}

// ------------------------------------------------------------------- scan
// As the fp32 step scan (16 channels x 16 lanes per block, quad-layout state
// and parameters), with bf16 32-blocked u, z, rows and y.
// One thread per (lane, channel), a block of 16 lanes x 16 channels.  The
// block's x_proj rows (as floats) and its channels' parameters go to shared
// memory, so that a thread's registers hold little beyond its state (d_state
// 32: 128 VGPRs with rows and parameters in registers, four waves per SIMD,
// for a kernel bound by moving the state).  Every thread issues the same
// number of row and parameter loads (the last ones repeat the first), then
// its state, u and z loads, which stay in flight across the barrier.
template <int DS, int RB, bool CACHED>
__global__ __launch_bounds__(256) void dec_b16_scan_kernel(LayerW Lw, const float* __restrict__ na_q,
                                                           const float* __restrict__ wdt_q,
                                                           const uint16_t* __restrict__ zt,
                                                           const uint16_t* __restrict__ cvt,
                                                           const uint16_t* __restrict__ rows,
                                                           float* ssm, uint16_t* yt, int M, int ld,
                                                           int ld_state, int r) {
  constexpr int NB = (RB + 2 * DS + 31) / 32;    // 32-feature blocks of an x_proj row
  constexpr int RW = NB * 32;                    // floats of a row in shared memory
  constexpr int NR = 16 * NB * 4;                // 16-byte row loads of the block
  constexpr int NP = scan_lds_floats<DS, RB>() / 4;  // 16-byte parameter loads
  constexpr int PER = (NR + NP + 255) / 256;     // loads per thread
  static_assert(PER * 256 - (NR + NP) <= NR + NP, "repeated loads fall in range");
  __shared__ __align__(16) float rowf[16 * RW];
  __shared__ __align__(16) float4 par[NP];
  const int tid = threadIdx.x, cl = tid & 15, lm = tid >> 4;
  const int cb = blockIdx.y;
  const int c = cb * 16 + cl;
  const int m0 = blockIdx.x * 16;
  const int m = m0 + lm, mc = min(m, M - 1);
  const u32x4* R4 = reinterpret_cast<const u32x4*>(rows);
  // 1. rows and parameters
  u32x4 v[PER];
  int slot[PER];
#pragma unroll
  for (int k = 0; k < PER; ++k) {
    int q = tid + 256 * k;
    q = q < NR + NP ? q : q - (NR + NP);
    slot[k] = q;
    const u32x4* src;
    if (q < NR) {
      const int rl = q / (NB * 4), kb = (q / 4) % NB, q4 = q % 4;
      src = R4 + ((size_t)kb * ld + min(m0 + rl, M - 1)) * 4 + q4;
    } else {
      src = reinterpret_cast<const u32x4*>(scan_lds_src<DS, RB>(Lw, na_q, wdt_q, cb, q - NR));
    }
    v[k] = *src;
  }
  // 2. the state, u and z (lane mc), in flight across the barrier
  float h[DS];
  float4* h4 = reinterpret_cast<float4*>(ssm);
#pragma unroll
  for (int n4 = 0; n4 < DS / 4; ++n4) {
    const float4 hv = state_ld4(h4 + ((size_t)(cb * (DS / 4) + n4) * ld_state + mc) * 16 + cl, CACHED);
    h[4 * n4] = hv.x; h[4 * n4 + 1] = hv.y; h[4 * n4 + 2] = hv.z; h[4 * n4 + 3] = hv.w;
  }
  const size_t cm = dblk32(c, mc, ld);
  const uint16_t ub = cvt[cm], zb = zt[cm];
  // 3. rows (bf16 pairs to floats: feature 2 e of a word in its low half) and
  // parameters to shared memory
#pragma unroll
  for (int k = 0; k < PER; ++k) {
    const int q = slot[k];
    if (q < NR) {
      const int rl = q / (NB * 4), kb = (q / 4) % NB, q4 = q % 4;
      float* o = rowf + rl * RW + 32 * kb + 8 * q4;
      reinterpret_cast<float4*>(o)[0] = make_float4(u2f(v[k][0] << 16), u2f(v[k][0] & 0xFFFF0000u),
                                                    u2f(v[k][1] << 16), u2f(v[k][1] & 0xFFFF0000u));
      reinterpret_cast<float4*>(o)[1] = make_float4(u2f(v[k][2] << 16), u2f(v[k][2] & 0xFFFF0000u),
                                                    u2f(v[k][3] << 16), u2f(v[k][3] & 0xFFFF0000u));
    } else {
      par[q - NR] = make_float4(u2f(v[k][0]), u2f(v[k][1]), u2f(v[k][2]), u2f(v[k][3]));
    }
  }
  // LDS barrier without the fence of __syncthreads, which would also wait
  // for the state loads: this wave's shared-memory stores are done at
  // lgkmcnt(0)
  asm volatile("s_waitcnt lgkmcnt(0)\n\ts_barrier" ::: "memory");
  if (m >= M) return;  // after the block's only barrier
  const float* row = rowf + lm * RW;
  const float y = scan_token_p<DS, RB, MATH_HW>(
      h, ScanLds<DS, RB>{reinterpret_cast<const float*>(par), cl}, row, row + RB, r,
      bf16_to_f32(ub), bf16_to_f32(zb));
  yt[dblk32(c, m, ld)] = f32_to_bf16(y);
#pragma unroll
  for (int n4 = 0; n4 < DS / 4; ++n4)
    state_st4(h4 + ((size_t)(cb * (DS / 4) + n4) * ld_state + m) * 16 + cl,
              make_float4(h[4 * n4], h[4 * n4 + 1], h[4 * n4 + 2], h[4 * n4 + 3]), CACHED);
}

hipError_t launch_dec_b16_scan(const Dims& D, const LayerW& Lw, const float* na_q,
                               const float* wdt_q, const uint16_t* zt, const uint16_t* cvt,
                               const uint16_t* rows, float* ssm, uint16_t* yt, int M, int ld,
                               int ld_state, bool state_cached, hipStream_t s) {
  if (D.di % 16 || dec_rb(D.r) < D.r) return hipErrorInvalidValue;
  dim3 grid((M + 15) / 16, D.di / 16);
#define BOA_B16_SCAN(DSv, RBv)                                                                  \
  if (state_cached)                                                                             \
    BOA_LAUNCH((dec_b16_scan_kernel<DSv, RBv, true>), grid, dim3(256), 0, s, Lw, na_q,    \
                       wdt_q, zt, cvt, rows, ssm, yt, M, ld, ld_state, D.r);                     \
  else                                                                                          \
    BOA_LAUNCH((dec_b16_scan_kernel<DSv, RBv, false>), grid, dim3(256), 0, s, Lw, na_q,   \
                       wdt_q, zt, cvt, rows, ssm, yt, M, ld, ld_state, D.r)
  const int rb = dec_rb(D.r);
  if (D.ds == 16) {
    if (rb == 8) BOA_B16_SCAN(16, 8);
    else if (rb == 16) BOA_B16_SCAN(16, 16);
    else BOA_B16_SCAN(16, 32);
  } else if (D.ds == 32) {
    if (rb == 8) BOA_B16_SCAN(32, 8);
    else if (rb == 16) BOA_B16_SCAN(32, 16);
    else BOA_B16_SCAN(32, 32);
  } else {
    return hipErrorInvalidValue;
  }
#undef BOA_B16_SCAN
  return hipGetLastError();
}

}  // namespace boa
