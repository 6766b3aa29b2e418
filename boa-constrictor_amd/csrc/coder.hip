// Deterministic integer CDFs and the 64-bit range coder (one chunk per lane).
//
// CDF (portability_solved_cpp/range_coder_kernels.cu:504-561, 856-932): a
// 32-lane group per token, lane l owning symbols 8l..8l+7.  Max by the
// shuffle-down tree; e_j = exp((l_j - max) / T) in fp32; per-lane sequential
// double sum; total by the shuffle-down tree (lane 0's value broadcast);
// exclusive lane prefix by the Hillis-Steele shuffle-up scan; running double
// sums per lane; then the lane-boundary monotonicity fix-up, propagated lane
// by lane so that every frequency stays >= 1 (the reference's lock-step
// fix-up, :903-913, can leave a zero-frequency symbol when two adjacent lanes
// both shift; the two agree whenever the lock-step result is monotone).
// s_cdf is written to LDS once.  Symbol k's integer interval is
// low_k = floor(s_cdf[k] (2^24-256)) + k, high_k = low_{k+1} (2^24 for 255).
// On wave64 each wavefront carries two tokens, one per 32-lane half.
//
// Coder (range_coder_kernels.cu:46-60, 279-335, 572-627, 934-964): u64
// lower/range state, 32-bit words, 24-bit precision, inverted-run carry
// handling; decoder target q = min((point-lower)/(range>>24), 2^24-1).
#include "coder_device.h"

namespace boa {

__global__ __launch_bounds__(256) void cdf_rows_kernel(const float* __restrict__ logits,
                                                       const float* __restrict__ bias, float inv_t,
                                                       int rows, uint32_t* qcdf) {
  __shared__ double s_cdf[8][260];
  const int half = threadIdx.x >> 5, l = threadIdx.x & 31;
  const int row = blockIdx.x * 8 + half;
  const int rr = row < rows ? row : rows - 1;
  cdf_halfwave(logits + (size_t)rr * 256, bias, inv_t, s_cdf[half], l);
  if (row < rows) {
    uint32_t* q = qcdf + (size_t)row * 257;
#pragma unroll
    for (int i = 0; i < 8; ++i) q[8 * l + i] = q_low(s_cdf[half], 8 * l + i);
    if (l == 0) q[256] = TOTAL;
  }
}

// Integer CDF of a probability row the way the Python GPU codec builds it
// (gpu_range_coder.py:57-79, build_cdf_fast): free weight 2^24 - K, the row
// sum and the running sum in double in index order, low(i) =
// trunc(running * (free / sum)) + i, low(K) = 2^24; a row whose sum is not
// positive and finite gets the uniform CDF.  One thread per row (a plug-in
// for probabilities computed elsewhere, not the codec's hot path).  A
// negative scaled running sum, which valid probabilities never produce, is
// taken as 0 here where the reference's conversion is undefined.
__global__ void cdf_probs_kernel(const float* __restrict__ probs, int rows, int K,
                                 uint32_t* __restrict__ out) {
  const int r = blockIdx.x * blockDim.x + threadIdx.x;
  if (r >= rows) return;
  const float* p = probs + (size_t)r * K;
  uint32_t* c = out + (size_t)r * (K + 1);
  const uint32_t free_w = TOTAL - (uint32_t)K;
  double norm = 0.0;
  for (int i = 0; i < K; ++i) norm += (double)p[i];
  if (!(norm > 0.0) || !__builtin_isfinite(norm)) {
    const uint32_t step = free_w / (uint32_t)K + 1u;
    uint32_t acc = 0;
    for (int i = 0; i < K; ++i) {
      c[i] = acc;
      acc += step;
    }
  } else {
    const double scale = (double)free_w / norm;
    double cum = 0.0;
    for (int i = 0; i < K; ++i) {
      const double v = cum * scale;
      c[i] = (uint32_t)(v > 0.0 ? v : 0.0) + (uint32_t)i;
      cum += (double)p[i];
    }
  }
  c[K] = TOTAL;
}

hipError_t launch_cdf_probs(const float* probs, int rows, int K, uint32_t* out, hipStream_t s) {
  if (rows < 1 || K < 1 || K > 1024) return hipErrorInvalidValue;
  BOA_LAUNCH(cdf_probs_kernel, dim3((rows + 63) / 64), dim3(64), 0, s, probs, rows, K, out);
  return hipGetLastError();
}

hipError_t launch_cdf_rows(const float* logits, const float* bias, float inv_temp, int rows,
                           uint32_t* qcdf, hipStream_t s) {
  BOA_LAUNCH(cdf_rows_kernel, dim3((rows + 7) / 8), dim3(256), 0, s, logits, bias, inv_temp,
                     rows, qcdf);
  return hipGetLastError();
}

// ---------------------------------------------------------------- encode
__global__ void rc_enc_init_kernel(RcEnc* st, int lanes) {
  const int b = blockIdx.x * blockDim.x + threadIdx.x;
  if (b >= lanes) return;
  RcEnc e;
  e.lower = 0; e.range = ~0ull; e.inverted_num = 0; e.first_inv_lower_word = 0;
  e.write_idx_words = 0; e.pad_ = 0;
  st[b] = e;
}

hipError_t launch_rc_enc_init(RcEnc* st, int lanes, hipStream_t s) {
  BOA_LAUNCH(rc_enc_init_kernel, dim3((lanes + 255) / 256), dim3(256), 0, s, st, lanes);
  return hipGetLastError();
}

// One thread per lane codes positions t in [t0, min(t0+T, len_b - 1)): the
// prediction made at t for byte t+1 (range_coder_kernels.cu:854-858 with
// boa.cpp:463-468's per-tile bound).
__global__ void rc_encode_tile_kernel(const uint2* __restrict__ lowprob, TokenSrc tok, int T,
                                      int t0, int lanes, RcEnc* states, uint32_t* out,
                                      int64_t pitch_words) {
  const int b = blockIdx.x * blockDim.x + threadIdx.x;
  if (b >= lanes) return;
  int64_t len = tok.total - (int64_t)b * tok.stride;
  len = len < 0 ? 0 : (len > tok.len ? tok.len : len);
  int64_t end = len - 1;
  if (end > (int64_t)t0 + T) end = (int64_t)t0 + T;
  if (end <= t0) return;
  RcEnc st = states[b];
  uint32_t* o = out + (size_t)b * pitch_words;
  const uint2* lp = lowprob + (size_t)b * T;
  // The coder state is the only serial dependence: the (low, prob) pairs
  // are read EPF positions ahead, one batch in flight while the previous
  // batch is coded, so a lane waits on memory once per batch instead of
  // once per symbol.
  constexpr int EPF = 16;
  const int n = (int)(end - t0);
  uint2 cur[EPF], nxt[EPF];
#pragma unroll
  for (int i = 0; i < EPF; ++i) cur[i] = i < n ? lp[i] : make_uint2(0u, 0u);
  for (int q = 0; q < n; q += EPF) {
#pragma unroll
    for (int i = 0; i < EPF; ++i) nxt[i] = q + EPF + i < n ? lp[q + EPF + i] : make_uint2(0u, 0u);
#pragma unroll
    for (int i = 0; i < EPF; ++i)
      if (q + i < n) enc_put(st, cur[i].x, cur[i].y, o);
#pragma unroll
    for (int i = 0; i < EPF; ++i) cur[i] = nxt[i];
  }
  states[b] = st;
}

hipError_t launch_rc_encode_tile(const uint2* lowprob, TokenSrc tok, int T, int t0, int lanes,
                                 RcEnc* st, uint32_t* out, int64_t pitch_words, hipStream_t s) {
  BOA_LAUNCH(rc_encode_tile_kernel, dim3((lanes + 63) / 64), dim3(64), 0, s, lowprob, tok, T,
                     t0, lanes, st, out, pitch_words);
  return hipGetLastError();
}

__global__ void rc_finish_kernel(RcEnc* states, uint32_t* out, int64_t pitch_words,
                                 int32_t* sizes_words, int lanes) {
  const int b = blockIdx.x * blockDim.x + threadIdx.x;
  if (b >= lanes) return;
  RcEnc st = states[b];
  sizes_words[b] = enc_finish(st, out + (size_t)b * pitch_words);
  states[b] = st;
}

hipError_t launch_rc_finish(RcEnc* st, uint32_t* out, int64_t pitch_words, int32_t* sizes_words,
                            int lanes, hipStream_t s) {
  BOA_LAUNCH(rc_finish_kernel, dim3((lanes + 255) / 256), dim3(256), 0, s, st, out,
                     pitch_words, sizes_words, lanes);
  return hipGetLastError();
}

// ------------------------------------------------------------ compaction
// Exclusive prefix sum of the per-lane word counts (one 1024-thread block:
// wavefront inclusive scans, then a scan of the 16 wave totals, carried
// across 1024-lane slices), followed by a copy of every lane's words to its
// offset in the contiguous payload.
__global__ __launch_bounds__(1024) void scan_sizes_kernel(const int32_t* sizes, int lanes,
                                                          uint64_t* offsets) {
  __shared__ uint64_t wave_tot[16];
  __shared__ uint64_t carry;
  const int tid = threadIdx.x, lane = tid & 63, wave = tid >> 6;
  if (tid == 0) carry = 0;
  __syncthreads();
  for (int base = 0; base < lanes; base += 1024) {
    const int i = base + tid;
    const uint64_t v = i < lanes ? (uint64_t)sizes[i] : 0ull;
    uint64_t inc = v;
#pragma unroll
    for (int off = 1; off < 64; off <<= 1) {
      const uint64_t t = __shfl_up(inc, off, 64);
      if (lane >= off) inc += t;
    }
    if (lane == 63) wave_tot[wave] = inc;
    __syncthreads();
    uint64_t wbase = 0;
    for (int w = 0; w < wave; ++w) wbase += wave_tot[w];
    const uint64_t c = carry;
    if (i < lanes) offsets[i] = c + wbase + inc - v;
    __syncthreads();
    if (tid == 1023) carry = c + wbase + inc;
    __syncthreads();
  }
}

__global__ __launch_bounds__(256) void compact_kernel(const uint32_t* __restrict__ words,
                                                      int64_t pitch_words,
                                                      const int32_t* __restrict__ sizes,
                                                      const uint64_t* __restrict__ offsets,
                                                      uint32_t* payload) {
  const int b = blockIdx.y;
  const int n = sizes[b];
  const uint32_t* src = words + (size_t)b * pitch_words;
  uint32_t* dst = payload + offsets[b];
  for (int i = blockIdx.x * blockDim.x + threadIdx.x; i < n; i += gridDim.x * blockDim.x)
    dst[i] = src[i];
}

hipError_t launch_compact(const uint32_t* words, int64_t pitch_words, const int32_t* sizes_words,
                          int lanes, uint64_t* offsets_words, uint32_t* payload, hipStream_t s) {
  if (lanes <= 0) return hipSuccess;
  BOA_LAUNCH(scan_sizes_kernel, dim3(1), dim3(1024), 0, s, sizes_words, lanes,
                     offsets_words);
  hipError_t e = hipGetLastError();
  if (e != hipSuccess) return e;
  BOA_LAUNCH(compact_kernel, dim3(16, lanes), dim3(256), 0, s, words, pitch_words,
                     sizes_words, offsets_words, payload);
  return hipGetLastError();
}

// Warm-start compaction leaves streams in lane-iteration order; this moves
// stream i (sizes[i] words at src + src_off[i]) to dst + dst_off[i], one
// block per stream at a time.
__global__ __launch_bounds__(256) void gather_streams_kernel(const uint32_t* __restrict__ src,
                                                             const uint64_t* __restrict__ src_off,
                                                             const uint64_t* __restrict__ dst_off,
                                                             const int32_t* __restrict__ sizes,
                                                             int64_t n, uint32_t* __restrict__ dst) {
  for (int64_t i = blockIdx.x; i < n; i += gridDim.x) {
    const uint32_t* a = src + src_off[i];
    uint32_t* b = dst + dst_off[i];
    for (int k = threadIdx.x; k < sizes[i]; k += blockDim.x) b[k] = a[k];
  }
}

hipError_t launch_gather_streams(const uint32_t* src, const uint64_t* src_off,
                                 const uint64_t* dst_off, const int32_t* sizes, int64_t n,
                                 uint32_t* dst, hipStream_t s) {
  if (n <= 0) return hipSuccess;
  const unsigned blocks = (unsigned)(n < 8192 ? n : 8192);
  BOA_LAUNCH(gather_streams_kernel, dim3(blocks), dim3(256), 0, s, src, src_off, dst_off,
                     sizes, n, dst);
  return hipGetLastError();
}

// ---------------------------------------------------------------- decode
__global__ void rc_dec_init_kernel(RcDec* st, const uint32_t* payload,
                                   const uint64_t* offsets_words, const int32_t* sizes_words,
                                   int lanes) {
  const int b = blockIdx.x * blockDim.x + threadIdx.x;
  if (b >= lanes) return;
  RcDec d;
  dec_init(d, payload + offsets_words[b], sizes_words[b]);
  st[b] = d;
}

hipError_t launch_rc_dec_init(RcDec* st, const uint32_t* payload, const uint64_t* offsets_words,
                              const int32_t* sizes_words, int lanes, hipStream_t s) {
  BOA_LAUNCH(rc_dec_init_kernel, dim3((lanes + 255) / 256), dim3(256), 0, s, st, payload,
                     offsets_words, sizes_words, lanes);
  return hipGetLastError();
}

// One 32-lane half-wave per lane: head bias, CDF, the first symbol whose
// interval holds the coder target (8 rounds of 32 candidates, ballot +
// first-set-bit as range_coder_kernels.cu:594-610), then the state update.
__global__ __launch_bounds__(256) void decode_step_kernel(
    const float* __restrict__ logits, const float* __restrict__ head_b2, float inv_t, uint8_t* tok,
    const int32_t* __restrict__ lens, const int* __restrict__ t_counter, uint8_t* out,
    int64_t out_stride, RcDec* states, const uint32_t* __restrict__ payload,
    const uint64_t* __restrict__ offsets_words, const int32_t* __restrict__ sizes_words,
    int lanes) {
  __shared__ double s_cdf[8][260];
  __shared__ uint32_t s_target[8];
  const int half = threadIdx.x >> 5, l = threadIdx.x & 31;
  const XcdSlot blk = xcd_slot(blockIdx.x, 8);  // 8 blocks of 8 lanes per 64-lane group
  if (blk.grp * 64 >= lanes) return;           // the whole block, before the barrier
  const int b = blk.grp * 64 + blk.j * 8 + half;
  const int bb = b < lanes ? b : lanes - 1;
  const int t = *t_counter;
  const bool active = b < lanes && t < lens[bb];
  cdf_halfwave(logits + (size_t)bb * 256, head_b2, inv_t, s_cdf[half], l);
  RcDec st;
  if (active && l == 0) {
    st = states[b];
    s_target[half] = dec_target(st);
  }
  __syncthreads();
  if (!active) return;  // no barrier follows
  int sym;
  uint32_t low_s, high_s;
  cdf_search_halfwave(s_cdf[half], s_target[half], l, sym, low_s, high_s);
  if (l == 0) {
    const uint32_t* in = payload + offsets_words[b];
    dec_advance(st, low_s, high_s, in, sizes_words[b]);
    states[b] = st;
    out[(size_t)b * out_stride + t] = (uint8_t)sym;
    tok[b] = (uint8_t)sym;
  }
}

hipError_t launch_decode_step(const float* logits, const float* head_b2, float inv_temp,
                              uint8_t* tok, const int32_t* lens, const int* t_counter,
                              uint8_t* out, int64_t out_stride, RcDec* st, const uint32_t* payload,
                              const uint64_t* offsets_words, const int32_t* sizes_words, int lanes,
                              hipStream_t s) {
  BOA_LAUNCH(decode_step_kernel, dim3(xcd_grid(lanes, 8)), dim3(256), 0, s, logits, head_b2,
                     inv_temp, tok, lens, t_counter, out, out_stride, st, payload, offsets_words,
                     sizes_words, lanes);
  return hipGetLastError();
}

// ------------------------------------------------- explicit-CDF test hooks
__global__ void rc_encode_cdf_kernel(const uint32_t* __restrict__ cdf, const uint8_t* syms,
                                     int n_sym, int lanes, uint32_t* out, int64_t pitch_words,
                                     int32_t* sizes_words) {
  const int b = blockIdx.x * blockDim.x + threadIdx.x;
  if (b >= lanes) return;
  RcEnc st;
  st.lower = 0; st.range = ~0ull; st.inverted_num = 0; st.first_inv_lower_word = 0;
  st.write_idx_words = 0; st.pad_ = 0;
  uint32_t* o = out + (size_t)b * pitch_words;
  for (int i = 0; i < n_sym; ++i) {
    const uint32_t* c = cdf + ((size_t)b * n_sym + i) * 257;
    const uint32_t s = syms[(size_t)b * n_sym + i];
    enc_put(st, c[s], c[s + 1] - c[s], o);
  }
  sizes_words[b] = enc_finish(st, o);
}

hipError_t launch_rc_encode_cdf(const uint32_t* cdf, const uint8_t* syms, int n_sym, int lanes,
                                uint32_t* out, int64_t pitch_words, int32_t* sizes_words,
                                hipStream_t s) {
  BOA_LAUNCH(rc_encode_cdf_kernel, dim3((lanes + 63) / 64), dim3(64), 0, s, cdf, syms, n_sym,
                     lanes, out, pitch_words, sizes_words);
  return hipGetLastError();
}

__global__ void rc_decode_cdf_kernel(const uint32_t* __restrict__ cdf, int n_sym, int lanes,
                                     const uint32_t* in, int64_t pitch_words,
                                     const int32_t* sizes_words, uint8_t* syms) {
  const int b = blockIdx.x * blockDim.x + threadIdx.x;
  if (b >= lanes) return;
  RcDec st;
  const uint32_t* src = in + (size_t)b * pitch_words;
  dec_init(st, src, sizes_words[b]);
  for (int i = 0; i < n_sym; ++i) {
    const uint32_t* c = cdf + ((size_t)b * n_sym + i) * 257;
    const uint32_t q = dec_target(st);
    int s = 0;
    uint32_t lo = 0, hi = 0;
    for (int k = 0; k < 256; ++k)
      if (q >= c[k] && q < c[k + 1]) { s = k; lo = c[k]; hi = c[k + 1]; break; }
    syms[(size_t)b * n_sym + i] = (uint8_t)s;
    dec_advance(st, lo, hi, src, sizes_words[b]);
  }
}

hipError_t launch_rc_decode_cdf(const uint32_t* cdf, int n_sym, int lanes, const uint32_t* in,
                                int64_t pitch_words, const int32_t* sizes_words, uint8_t* syms,
                                hipStream_t s) {
  BOA_LAUNCH(rc_decode_cdf_kernel, dim3((lanes + 63) / 64), dim3(64), 0, s, cdf, n_sym,
                     lanes, in, pitch_words, sizes_words, syms);
  return hipGetLastError();
}

}  // namespace boa
