// Device-side range coder and CDF helpers, shared by the coder kernels and
// the persistent decode kernel.  The algorithms and their reference lines
// are described at the top of coder.hip.
#pragma once
#include "boa_kernels.h"

namespace boa {

constexpr uint32_t TOTAL = 1u << 24;
constexpr double CDF_SCALE = (double)((1u << 24) - 256u);

// ----------------------------------------------------------------- coder
__device__ __forceinline__ void enc_put(RcEnc& st, uint32_t left, uint32_t prob, uint32_t* out) {
  if (prob == 0) prob = 1;
  const uint64_t scale = st.range >> 24;
  const uint64_t old_lower = st.lower;
  st.range = scale * (uint64_t)prob;
  st.lower = st.lower + scale * (uint64_t)left;
  if (st.inverted_num > 0) {
    const uint64_t sum = st.lower + st.range;
    if (sum > st.lower) {
      const bool carry = st.lower < old_lower;
      const uint32_t first = carry ? st.first_inv_lower_word + 1u : st.first_inv_lower_word;
      const uint32_t rest = carry ? 0u : 0xFFFFFFFFu;
      out[st.write_idx_words++] = first;
      for (int k = 1; k < st.inverted_num; ++k) out[st.write_idx_words++] = rest;
      st.inverted_num = 0;
    }
  }
  // range >= 2^32 before the update gives range >= 2^8 after it, so one
  // shift always restores the invariant; the bound of two keeps a corrupted
  // state from spinning.
  for (int it = 0; it < 2 && st.range < (1ull << 32); ++it) {
    const uint32_t lower_word = (uint32_t)(st.lower >> 32);
    st.lower <<= 32;
    st.range <<= 32;
    if (st.inverted_num > 0) {
      st.inverted_num++;
    } else {
      const uint64_t sum = st.lower + st.range;
      if (sum > st.lower) {
        out[st.write_idx_words++] = lower_word;
      } else {
        st.inverted_num = 1;
        st.first_inv_lower_word = lower_word;
      }
    }
  }
}

__device__ __forceinline__ int32_t enc_finish(RcEnc& st, uint32_t* out) {
  if (st.range == ~0ull) return 0;
  const uint64_t point = st.lower + ((1ull << 32) - 1ull);
  if (st.inverted_num > 0) {
    const bool carry = point < st.lower;
    const uint32_t first = carry ? st.first_inv_lower_word + 1u : st.first_inv_lower_word;
    const uint32_t rest = carry ? 0u : 0xFFFFFFFFu;
    out[st.write_idx_words++] = first;
    for (int k = 1; k < st.inverted_num; ++k) out[st.write_idx_words++] = rest;
    st.inverted_num = 0;
  }
  const uint32_t point_word = (uint32_t)(point >> 32);
  out[st.write_idx_words++] = point_word;
  const uint64_t upper = st.lower + st.range;
  if ((uint32_t)(upper >> 32) == point_word) out[st.write_idx_words++] = 0u;
  return st.write_idx_words;
}

__device__ __forceinline__ void dec_init(RcDec& st, const uint32_t* in, int32_t n_words) {
  st.lower = 0;
  st.range = ~0ull;
  st.point = 0;
  st.read_idx_words = 0;
  st.pad_ = 0;
  for (int k = 0; k < 2; ++k) {
    const uint32_t w = (st.read_idx_words < n_words) ? in[st.read_idx_words++] : 0u;
    st.point = (st.point << 32) | (uint64_t)w;
  }
}

__device__ __forceinline__ uint32_t dec_target(const RcDec& st) {
  const uint64_t scale = st.range >> 24;
  uint64_t q = (st.point - st.lower) / scale;
  if (q >= TOTAL) q = TOTAL - 1;
  return (uint32_t)q;
}

__device__ __forceinline__ void dec_advance(RcDec& st, uint32_t low, uint32_t high,
                                            const uint32_t* in, int32_t n_words) {
  const uint64_t scale = st.range >> 24;
  uint32_t prob = high - low;
  if (prob == 0) prob = 1;
  st.lower = st.lower + scale * (uint64_t)low;
  st.range = scale * (uint64_t)prob;
  for (int it = 0; it < 2 && st.range < (1ull << 32); ++it) {
    st.lower <<= 32;
    st.range <<= 32;
    const uint32_t w = (st.read_idx_words < n_words) ? in[st.read_idx_words++] : 0u;
    st.point = (st.point << 32) | (uint64_t)w;
  }
}

// dec_advance for a decoder that keeps running across steps in registers:
// nw holds the word at read_idx_words (0 past the end), loaded when the
// previous word was taken, so the load's latency overlaps the steps between
// two renormalisations.  The state sequence is dec_advance's.
__device__ __forceinline__ void dec_advance_ahead(RcDec& st, uint32_t low, uint32_t high,
                                                  const uint32_t* in, int32_t n_words,
                                                  uint32_t& nw) {
  const uint64_t scale = st.range >> 24;
  uint32_t prob = high - low;
  if (prob == 0) prob = 1;
  st.lower = st.lower + scale * (uint64_t)low;
  st.range = scale * (uint64_t)prob;
  for (int it = 0; it < 2 && st.range < (1ull << 32); ++it) {
    st.lower <<= 32;
    st.range <<= 32;
    const uint32_t w = nw;
    if (st.read_idx_words < n_words) ++st.read_idx_words;
    nw = st.read_idx_words < n_words ? in[st.read_idx_words] : 0u;
    st.point = (st.point << 32) | (uint64_t)w;
  }
}

// ------------------------------------------------------------------- CDF
// The cumulative probabilities of one logits row `lg` on a half-wave: lane
// l ends with the exclusive running sums r[i] of symbols 8l + i.
__device__ __forceinline__ void cdf_halfwave_regs(const float* lg, const float* bias, float inv_t,
                                                  int l, double (&r)[8]) {
  float v[8];
  float mx = -1e30f;
#pragma unroll
  for (int i = 0; i < 8; ++i) {
    const int c = 8 * l + i;
    const float val = bias ? lg[c] + bias[c] : lg[c];
    v[i] = val;
    mx = fmaxf(mx, val);
  }
#pragma unroll
  for (int off = 16; off > 0; off >>= 1) mx = fmaxf(mx, __shfl_down(mx, off, 32));
  mx = __shfl(mx, 0, 32);
  double sd = 0.0;
#pragma unroll
  for (int i = 0; i < 8; ++i) {
    const float e = exp2_neg(((v[i] - mx) * inv_t) * 1.44269504088896340736f);
    v[i] = e;
    sd += (double)e;
  }
  double tot = sd;
#pragma unroll
  for (int off = 16; off > 0; off >>= 1) tot = tot + __shfl_down(tot, off, 32);
  tot = __shfl(tot, 0, 32);
  const double inv = 1.0 / tot;
  const double ts = sd * inv;
  double pre = ts;
#pragma unroll
  for (int off = 1; off <= 16; off <<= 1) {
    const double tmp = __shfl_up(pre, off, 32);
    if (l >= off) pre = pre + tmp;
  }
  double run = pre - ts;
#pragma unroll
  for (int i = 0; i < 8; ++i) {
    r[i] = run;
    run += (double)v[i] * inv;
  }
  // Lane-boundary monotonicity fix-up, propagated lane by lane: lane j
  // compares its first entry with lane j-1's already fixed last entry and
  // shifts its eight entries up by the difference.  When no lane starts below
  // its left neighbour's (unfixed) last entry nothing changes, which the
  // ballot detects without running the chain.
  double last = r[7];
  const double left_last = __shfl_up(last, 1, 32);
  const bool need = l > 0 && r[0] < left_last;
  const int shift = threadIdx.x & 32;
  if ((uint32_t)(__ballot(need) >> shift) != 0u) {
    for (int j = 1; j < 32; ++j) {
      const double prev_last = __shfl(last, j - 1, 32);
      if (l == j && r[0] < prev_last) {
        const double delta = prev_last - r[0];
#pragma unroll
        for (int i = 0; i < 8; ++i) r[i] += delta;
        last = r[7];
      }
    }
  }
}

// The same into LDS.  Every thread of the block must call this (it contains
// a block barrier).  `s_cdf` is this half-wave's 257-entry LDS region.
__device__ __forceinline__ void cdf_halfwave(const float* lg, const float* bias, float inv_t,
                                             double* s_cdf, int l) {
  double r[8];
  cdf_halfwave_regs(lg, bias, inv_t, l, r);
#pragma unroll
  for (int i = 0; i < 8; ++i) s_cdf[8 * l + i] = r[i];
  if (l == 31) s_cdf[256] = 1.0;
  __syncthreads();
}

// Entry k of a half-wave's cumulative row held in registers (lane k / 8,
// element k % 8), broadcast to every lane of the half-wave.
__device__ __forceinline__ double cdf_entry(const double (&r)[8], int k) {
  const int e = k & 7;
  double mine = r[0];
#pragma unroll
  for (int i = 1; i < 8; ++i) mine = e == i ? r[i] : mine;
  return __shfl(mine, k >> 3, 32);
}

// The coder's (low, prob) of the byte that follows row `row` of a compress
// tile (row = lane b x T + t, position t0 + t of lane b's chunk; past the
// chunk's end the byte is 0), from the row's logits lg (bias already added),
// run by the row's half-wave (lane l) in the fused head.2 + CDF GEMM
// epilogues.  Rows at or past M store nothing.
__device__ __forceinline__ void cdf_row_lowprob(const float* lg, const CdfEpi& c, int row, int M,
                                                int l) {
  const int rr = row < M ? row : M - 1;
  double cr[8];
  cdf_halfwave_regs(lg, nullptr, c.inv_t, l, cr);
  const int b = rr / c.T, t = rr % c.T;
  const int64_t pic = (int64_t)c.t0 + t + 1;
  const int64_t pos = (int64_t)b * c.tok_stride + pic;
  const int sym = (pic < c.tok_len && pos < c.tok_total) ? c.tok_base[pos] : 0;
  const double c_lo = cdf_entry(cr, sym);
  const double c_hi = cdf_entry(cr, sym + 1 > 255 ? 255 : sym + 1);
  if (row < M && l == 0) {
    const uint32_t lo = (uint32_t)(c_lo * CDF_SCALE) + (uint32_t)sym;
    const uint32_t hi = sym == 255 ? TOTAL : (uint32_t)(c_hi * CDF_SCALE) + (uint32_t)(sym + 1);
    c.lowprob[row] = make_uint2(lo, hi - lo);
  }
}

__device__ __forceinline__ uint32_t q_low(const double* s_cdf, int k) {
  return (uint32_t)(s_cdf[k] * CDF_SCALE) + (uint32_t)k;
}
__device__ __forceinline__ uint32_t q_high(const double* s_cdf, int k) {
  return k == 255 ? TOTAL : (uint32_t)(s_cdf[k + 1] * CDF_SCALE) + (uint32_t)(k + 1);
}

// The decoder's symbol search on a half-wave (range_coder_kernels.cu:594-610):
// the first symbol k whose integer interval [low_k, high_k) holds the
// coder target, in 8 rounds of 32 candidates, ballot + first set bit; the
// result is broadcast to the half-wave.
__device__ __forceinline__ void cdf_search_halfwave(const double* s_cdf, uint32_t target, int l,
                                                    int& sym, uint32_t& low_s, uint32_t& high_s) {
  sym = 0;
  low_s = 0;
  high_s = 0;
  const int shift = (threadIdx.x & 32);
  for (int round = 0; round < 8; ++round) {
    const int k = round * 32 + l;
    const uint32_t lo = q_low(s_cdf, k), hi = q_high(s_cdf, k);
    const bool match = target >= lo && target < hi;
    const uint32_t mask = (uint32_t)(__ballot(match) >> shift);
    if (mask != 0u) {
      const int winner = __ffs(mask) - 1;
      sym = __shfl(k, winner, 32);
      low_s = __shfl(lo, winner, 32);
      high_s = __shfl(hi, winner, 32);
      return;
    }
  }
}

}  // namespace boa
