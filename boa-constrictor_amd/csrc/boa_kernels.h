// Kernel-level interface of the MI355X codec path (internal to the library).
#pragma once
#include <hip/hip_ext.h>
#include <hip/hip_runtime.h>
#include <stdint.h>

#include "boa_math.h"

namespace boa {

// Per-launch timing for the host profiler: while `stop` is set, BOA_LAUNCH
// passes the events to the dispatch itself (hipExtLaunchKernelGGL), so they
// stamp the kernel's start and end without separate marker packets -- the
// same span rocprofv3 reports.  The first launch of a profiled call takes
// `start`, every launch `stop` (so a helper that launches two kernels is
// timed from the first start to the last end).  Host-side state of the
// calling thread; see timed() in boa_api.hip.
struct LaunchTiming {
  hipEvent_t start = nullptr, stop = nullptr;
  int launches = 0;
};
extern thread_local LaunchTiming g_launch_timing;

#define BOA_LAUNCH(K, GRID, BLOCK, SHM, STREAM, ...)                                         \
  do {                                                                                       \
    if (::boa::g_launch_timing.stop) {                                                       \
      hipEvent_t boa_start_ =                                                                \
          ::boa::g_launch_timing.launches++ == 0 ? ::boa::g_launch_timing.start : nullptr;   \
      hipExtLaunchKernelGGL(K, dim3(GRID), dim3(BLOCK), (std::uint32_t)(SHM), STREAM,        \
                            boa_start_, ::boa::g_launch_timing.stop, 0u, __VA_ARGS__);        \
    } else {                                                                                 \
      hipLaunchKernelGGL(K, GRID, BLOCK, SHM, STREAM, __VA_ARGS__);                          \
    }                                                                                        \
  } while (0)

// Workgroups are dispatched to the 8 XCDs, each with its own L2, round-robin
// by block index.  The decode step's kernels keep every 64-lane group on one
// XCD, so that one kernel's outputs for those lanes are read by the next
// kernel from the same L2: block b, of per_group blocks per group, gets group
// b % 8 + 8 ((b / 8) / per_group) and index (b / 8) % per_group in it.
struct XcdSlot {
  int grp, j;
};
__device__ __forceinline__ XcdSlot xcd_slot(int b, int per_group) {
  const int s = b >> 3;
  return XcdSlot{(b & 7) + 8 * (s / per_group), s % per_group};
}
// blocks covering `lanes` lanes in 64-lane groups of per_group blocks
inline unsigned xcd_grid(int lanes, int per_group) {
  return (unsigned)(((lanes + 511) / 512) * 8 * per_group);
}


enum { ACT_NONE = 0, ACT_GELU = 1, ACT_RELU = 2 };

struct GemmArgs {
  const float* X; int ldx;        // activations [M][K]
  const float* W; int ldw;        // weights [K][ldw], ldw >= round_up(N, 256), zero padded
  float* C; int ldc;              // output [M][ldc]
  const float* bias;              // [N] or null
  const float* res; int ldr;      // residual [M][ldr] or null (may alias C)
  int M, N, K, act;
};
hipError_t gemm_f32(const GemmArgs& a, hipStream_t s);
// the CDF epilogue's inputs: the tile's tokens, the row -> (lane, position)
// map (row = lane * T + t, position t0 + t) and the temperature
struct CdfEpi {
  const uint8_t* tok_base;  // see TokenSrc
  int64_t tok_stride, tok_total, tok_len;
  int T, t0;
  float inv_t;
  uint2* lowprob;           // [M] (low, prob) of the next byte per row
};
hipError_t gemm_f32_head_cdf(const GemmArgs& a, const CdfEpi& cdf, hipStream_t s);
// A 256-wide GEMM (out_proj, FF2 at d_model 256) with the following
// LayerNorm in its epilogue: LN2 (sequential per-row sums) of acc + bias, or
// LN1 (the 32-lane tree) of acc + bias + residual, whose un-normalised rows
// are also stored to C (the residual stream).  The normalised rows go to out.
struct LnEpi {
  const float* w;
  const float* b;
  float* out;
  int ldo;
  int mode;  // 1 = LN1, 2 = LN2
  int n;     // the LayerNorm's width (real features of the 256)
};
hipError_t gemm_f32_ln(const GemmArgs& a, const LnEpi& ln, hipStream_t s);
// Tile configuration gemm_f32 picks: 0 = 128x256 (bulk GEMMs of a compress
// tile), 1 = 128x64 (narrow compress GEMMs), 2 = 32x32 (decode-step sizes).
int gemm_f32_config(const GemmArgs& a);

// Encoder / decoder coder state (layout of RCState / RCDecState,
// portability_solved_cpp/gemm_gpu.hpp:115-121, 212-217, padded to 8 bytes).
struct RcEnc {
  uint64_t lower, range;
  int32_t inverted_num;
  uint32_t first_inv_lower_word;
  int32_t write_idx_words;
  int32_t pad_;
};
struct RcDec {
  uint64_t lower, range, point;
  int32_t read_idx_words;
  int32_t pad_;
};

// Token source for a tile: token(b, t) = base[b*stride + t0 + t] when that
// position lies inside lane b's chunk, else 0 (the zero padding boa.cpp:412
// gives the last, short chunk).
struct TokenSrc {
  const uint8_t* base;  // first byte of lane 0's chunk
  int64_t stride;       // bytes between lanes' chunks (a multiple of len with warm-start)
  int64_t total;        // valid bytes counted from base
  int64_t len;          // positions per lane's chunk; bytes past total read as 0
};

struct LayerW {
  const float *ln1_w, *ln1_b, *w_in, *b_in, *conv_w, *conv_b, *w_x, *w_dt, *b_dt, *na2, *dd,
      *w_out, *b_out, *ln2_w, *ln2_b, *w1, *b1, *w2, *b2;
};

// Model dimensions and padded weight strides.  A model of d_model dn runs at
// width d >= dn, the next width the kernels are built for: features dn .. d-1
// (and inner channels 2 dn .. 2 d-1 of each half of in_proj's output) hold
// zero weights, so their activations are zero, every GEMM's K-ordered chain
// ends in exact zero terms, and the LayerNorms divide by dn.  dt_rank r is
// dn's: ceil(dn / 16).
struct Dims {
  int d, L, di, r, ds, R;
  int dn;  // the model's own d_model (LayerNorm width); d = dn for the built widths
  int ld_in, ld_x, ld_out, ld_1, ld_2, ld_h1, ld_h2;
};

// LayerNorm of rows with the reference's 32-lane tree reduction order; when
// `tok` is set, row b*T+t is first filled from the embedding table (and x is
// written), which fuses the embedding lookup into layer 0's LN1.
// bf16 GEMM (precision 1): X bf16 [M][ldx], W bf16 [N_pad][ldw] (k contiguous,
// N_pad = round_up(N, 256), zero rows), fp32 accumulation and epilogue; C is
// fp32 or bf16 (c_bf16), C2 an optional bf16 copy of C, res an fp32 residual.
struct GemmB16Args {
  const uint16_t* X; int ldx;
  const uint16_t* W; int ldw;
  void* C; int ldc; int c_bf16;
  uint16_t* C2;
  const float* bias;
  const float* res; int ldr;
  int M, N, K, act;
};
hipError_t gemm_bf16(const GemmB16Args& a, hipStream_t s);
// head.2 of the bf16 compress pass (N = 256, act none, bias = head.2's)
// fused with the CDF: each row's (low, prob) of the next byte goes to
// cdf.lowprob and the logits are not stored (C unused)
hipError_t gemm_bf16_head_cdf(const GemmB16Args& a, const CdfEpi& cdf, hipStream_t s);
// FF1 + GELU + FF2 (+ b2 + residual) of the bf16 compress pass in one kernel:
// X bf16 [M][D] (LN2's output), W1 bf16 [4D][D], W2 bf16 [D][4D] (the
// gemm_bf16 layouts), res and C fp32 [M][D] (may alias), C2 an optional bf16
// copy of C.  D = 256.  With ln2_w/ln2_b, X is out_proj's output and LN2 is
// applied to it in the kernel; with xn (may alias X), the next layer's LN1
// of C (ln1_w, ln1_b) is stored there in bf16.
struct FfnB16Args {
  const uint16_t* X;
  const uint16_t* W1;
  const uint16_t* W2;
  const float* b1;
  const float* b2;
  const float* res;
  float* C;
  uint16_t* C2;
  int M, D;
  int n = 0;  // the LayerNorms' width (real features of the D; 0 = D)
  const float* ln2_w = nullptr;
  const float* ln2_b = nullptr;
  const float* ln1_w = nullptr;
  const float* ln1_b = nullptr;
  uint16_t* xn = nullptr;
};
hipError_t ffn_bf16(const FfnB16Args& a, hipStream_t s);
hipError_t launch_b16_weight_nk(const float* w, int ldw_in, int N, int K, int n_pad, uint16_t* out,
                                hipStream_t s);

// Activations other than the residual stream x are fp32, or bf16 (uint16_t)
// when `bf16` is set; x and the recurrent state are always fp32.
// Rows are d wide; the LayerNorms take the statistics of the first n.
hipError_t launch_ln1(const float* emb, TokenSrc tok, int T, int t0, float* x, void* xn,
                      const float* w, const float* b, int rows, int d, int n, bool bf16,
                      hipStream_t s);
// LayerNorm with sequential per-row sums (LN2 order), in place allowed.
hipError_t launch_ln2(const void* x, void* out, const float* w, const float* b, int rows, int d,
                      int n, bool bf16, hipStream_t s);
hipError_t launch_conv_chunk(const void* xz, float* conv_state, const float* w, const float* cb,
                             void* out, int lanes, int T, int di, bool bf16, hipStream_t s);
hipError_t launch_scan_chunk(const Dims& D, const LayerW& Lw, const void* xz, const void* conv,
                             const void* delta, float* ssm_state, void* y, int lanes, int T,
                             bool bf16, hipStream_t s);
hipError_t launch_fill_zero(void* p, size_t bytes, hipStream_t s);

// ---- decode step, features-major activations X^T[feature][lane] ----------
// Activations and weights are k-blocked (element (k, m) at
// ((k/16) ld + m) 16 + 4 (k%4) + (k%16)/4), see decode.hip.
struct DecGemmArgs {
  const float* Xt; int ldx;   // activations, k-blocked, lane capacity ldx
  const float* W; int ldw;    // weights, k-blocked over N columns, ldw >= round_up(N, 16)
  float* C; int ldc;          // output k-blocked over N (row_major = 0) or [M][ldc] (= 1)
  const float* bias;          // [N] or null
  const float* res; int ldr;  // residual, k-blocked, or null (may alias C)
  int M, N, K, act, row_major;
  // in_proj with the causal conv step fused: features n < conv_di run the
  // conv (state [n][ld_state] float4, output conv_out k-blocked); features
  // n >= conv_di are stored at C feature n - conv_di (the z half)
  int conv_di;
  float* conv_state; int ld_state;
  const float* conv_w; const float* conv_b; float* conv_out;
  int state_cached;  // conv state through the caches (1) or streamed (0)
  int ln_n;          // launch_dec_ln_gemm: the LayerNorm's width (real features of K)
};
hipError_t dec_gemm(const DecGemmArgs& a, hipStream_t s);
// LayerNorm (mode 1: LN1, mode 2: LN2; weights lw, lb) of the K = d features
// of a.Xt fused in front of the GEMM a (in_proj or FF1).  With emb, layer
// 0's LN1: rows are emb[tok[m]] and are also stored as x (k-blocked, xt),
// and *t_counter is incremented.  Needs d in {64, 128, 256} and N % 64 == 0.
bool dec_ln_gemm_fits(int d, int N);
hipError_t launch_dec_ln_gemm(int mode, const DecGemmArgs& a, const float* emb, const uint8_t* tok,
                              float* xt, const float* lw, const float* lb, int* t_counter,
                              hipStream_t s);
// decode GEMM with an explicit wave-tile configuration (4, 9, 10, 13 or 15; all give the same bits)
hipError_t dec_gemm_cfg(const DecGemmArgs& a, int cfg, hipStream_t s);
hipError_t launch_dec_weight_blk(const float* w, int ldw_in, int n_src, float* out, int K, int ldn,
                                 int permute, int zs, int ze, hipStream_t s);
hipError_t launch_dec_scan_params(const float* w_dt, const float* na, float* wdt_q, float* na_q,
                                  int r, int rb, int ds, int di, hipStream_t s);
// dt_rank slots of the decode scan's row (features [0, dec_rb) hold dt_in)
inline int dec_rb(int r) { return r <= 8 ? 8 : (r <= 16 ? 16 : 32); }
hipError_t launch_dec_ln1(const float* emb, const uint8_t* tok, float* xt, float* xnt,
                          const float* w, const float* b, int M, int d, int n, int ld,
                          int* t_counter, hipStream_t s);
hipError_t launch_dec_ln2(const float* xt, float* xnt, const float* w, const float* b, int M, int d,
                          int n, int ld, hipStream_t s);
// x_proj fused with the decode scan (dec_xscan_kernel); same results as
// dec_gemm (x_proj) + launch_dec_scan
bool dec_xscan_fits(const Dims& D);
hipError_t launch_dec_xscan(const Dims& D, const LayerW& Lw, const float* na_q, const float* wdt_q,
                            const float* w_x, int ldw_x, const float* zt, const float* cvt,
                            float* ssm, float* yt, int M, int ld, int ld_state, bool state_cached,
                            hipStream_t s);
hipError_t launch_dec_scan(const Dims& D, const LayerW& Lw, const float* na_q, const float* wdt_q,
                           const float* zt, const float* cvt, const float* rows, float* ssm, float* yt,
                           int M, int ld, int ld_state, bool state_cached, hipStream_t s);
// ---- persistent decode for small models (decode_persist.hip) -----------
// One block of 1024 threads per 16 lanes runs steps 1 .. maxlen-1 of a batch
// (model, CDF, search, coder) with the step kernels' operations and state
// layouts.  d_model 64, d_state 16, at most PERSIST_MAX_LAYERS layers (their
// per-channel parameters are staged in LDS).
constexpr int PERSIST_MAX_LAYERS = 2;
struct PersistLayer {
  const float *ln1_w, *ln1_b, *w_in, *b_in, *conv_w, *conv_b, *w_x, *na_q, *wdt_q, *b_dt, *dd,
      *w_out, *b_out, *ln2_w, *ln2_b, *w1, *b1, *w2, *b2;  // decode (k-blocked) weights
  float *conv, *ssm;                                         // step-layout state
};
struct PersistArgs {
  PersistLayer layer[PERSIST_MAX_LAYERS];
  int L, r, lanes, maxlen, ld_state;
  int ln_n;  // the LayerNorms' width (real features of the 64)
  const float *emb, *hw1, *hb1, *hw2, *hb2;
  float inv_t;
  uint8_t* tok;
  const int32_t* lens;
  int* t_counter;
  uint8_t* out;
  int64_t out_stride;
  RcDec* states;
  const uint32_t* payload;
  const uint64_t* offsets;
  const int32_t* sizes;
};
bool dec_persist_fits(int d, int ds, int r, int L);
// lanes per block: the fewest (4, 8, 16) whose grid fits n_cus workgroups
int dec_persist_lanes_per_block(int lanes, int n_cus);
hipError_t launch_dec_persist(const PersistArgs& a, int d, int ds, int n_cus, hipStream_t s);

// ---- decode step, bf16 precision (decode_bf16.hip) ----------------------
// Activations bf16 in the 32-blocked layout (feature k of lane m at
// ((k/32) ld + m) 32 + k%32), the residual stream fp32 k-blocked.
enum { DEC_OUT_B16 = 0, DEC_OUT_F32 = 1, DEC_OUT_ROWMAJOR = 2 };
struct DecB16Args {
  const uint16_t* X; int ldx;   // bf16 32-blocked activations
  const uint16_t* W; int ldw;   // bf16 32-blocked weights, ldw >= round_up(N, 16)
  void* C; int ldc; int out_mode;
  uint16_t* C2;                 // DEC_OUT_F32: optional bf16 32-blocked copy of C
  const float* bias;
  const float* res; int ldr;    // DEC_OUT_F32: fp32 k-blocked residual
  int M, N, K, act;
  int conv_di;                  // DEC_OUT_B16 in_proj: the conv step on features < conv_di
  float* conv_state; int ld_state;
  const float* conv_w; const float* conv_b; uint16_t* conv_out;
  int state_cached;             // conv state through the caches (1) or streamed (0)
  int n_cus;                    // the device's compute units (0: 256), for the block shape
};
hipError_t dec_b16_gemm(const DecB16Args& a, hipStream_t s);
hipError_t launch_dec_b16_weight(const float* w, int ldw_in, int n_src, uint16_t* out, int K,
                                 int ldn, int zs, int ze, hipStream_t s);
hipError_t launch_dec_b16_ln1(const float* emb, const uint8_t* tok, float* xt, uint16_t* xnt,
                              const float* w, const float* b, int M, int d, int n, int ld,
                              int* t_counter, hipStream_t s);
hipError_t launch_dec_b16_ln2(const uint16_t* src, uint16_t* xnt, const float* w, const float* b,
                              int M, int d, int n, int ld, hipStream_t s);
hipError_t launch_dec_b16_scan(const Dims& D, const LayerW& Lw, const float* na_q,
                               const float* wdt_q, const uint16_t* zt, const uint16_t* cvt,
                               const uint16_t* rows, float* ssm, uint16_t* yt, int M, int ld,
                               int ld_state, bool state_cached, hipStream_t s);

// chunk layout: conv [lane][c][4], ssm [lane][c][n]; step layout: conv
// [c][lane][4], ssm [c/16][n/4][lane][c%16][n%4] with lane stride ld_state.
// conv_b16: the step-layout conv state is four bf16 per channel and lane
// (bf16 precision), else four floats
hipError_t launch_state_relayout(const float* conv_in, const float* ssm_in, float* conv_out,
                                 float* ssm_out, int lanes, int di, int ds, int ld_state,
                                 bool to_step, bool conv_b16, hipStream_t s);

// CDF + coder kernels.
hipError_t launch_rc_enc_init(RcEnc* st, int lanes, hipStream_t s);
hipError_t launch_rc_encode_tile(const uint2* lowprob, TokenSrc tok, int T, int t0, int lanes,
                                 RcEnc* st, uint32_t* out, int64_t pitch_words, hipStream_t s);
hipError_t launch_rc_finish(RcEnc* st, uint32_t* out, int64_t pitch_words, int32_t* sizes_words,
                            int lanes, hipStream_t s);
hipError_t launch_compact(const uint32_t* words, int64_t pitch_words, const int32_t* sizes_words,
                          int lanes, uint64_t* offsets_words, uint32_t* payload, hipStream_t s);
hipError_t launch_gather_streams(const uint32_t* src, const uint64_t* src_off,
                                 const uint64_t* dst_off, const int32_t* sizes, int64_t n,
                                 uint32_t* dst, hipStream_t s);
hipError_t launch_rc_dec_init(RcDec* st, const uint32_t* payload, const uint64_t* offsets_words,
                              const int32_t* sizes_words, int lanes, hipStream_t s);
// head.2 (a: Xt = head.1 output, W = head.2 decode weights, N = 256, no
// bias, row-major) fused with launch_decode_step; same results as the two
hipError_t launch_dec_head_step(const DecGemmArgs& a, const float* head_b2, float inv_temp,
                                uint8_t* tok, const int32_t* lens, const int* t_counter,
                                uint8_t* out, int64_t out_stride, RcDec* st,
                                const uint32_t* payload, const uint64_t* offsets_words,
                                const int32_t* sizes_words, hipStream_t s);
hipError_t launch_decode_step(const float* logits, const float* head_b2, float inv_temp,
                              uint8_t* tok, const int32_t* lens, const int* t_counter,
                              uint8_t* out, int64_t out_stride, RcDec* st, const uint32_t* payload,
                              const uint64_t* offsets_words, const int32_t* sizes_words, int lanes,
                              hipStream_t s);
// Test hooks: quantised CDFs of logits rows, and coder runs on explicit CDFs.
// build_cdf_fast of the Python GPU codec: probs [rows][K] -> out [rows][K+1]
hipError_t launch_cdf_probs(const float* probs, int rows, int K, uint32_t* out, hipStream_t s);
hipError_t launch_cdf_rows(const float* logits, const float* bias, float inv_temp, int rows,
                           uint32_t* qcdf, hipStream_t s);
hipError_t launch_rc_encode_cdf(const uint32_t* cdf, const uint8_t* syms, int n_sym, int lanes,
                                uint32_t* out, int64_t pitch_words, int32_t* sizes_words,
                                hipStream_t s);
hipError_t launch_rc_decode_cdf(const uint32_t* cdf, int n_sym, int lanes, const uint32_t* in,
                                int64_t pitch_words, const int32_t* sizes_words, uint8_t* syms,
                                hipStream_t s);

}  // namespace boa
