/*
 * refcpu.c -- CPU restatement of BoaConstrictor's boa.cpp codec path.
 *
 * TEST INFRASTRUCTURE ONLY (parity oracle and timed CPU baseline).  See
 * refcpu.h for the list of reference lines each part follows.  Built with
 * -ffp-contract=off: every fused multiply-add below is an explicit fmaf().
 */
#include "refcpu.h"

#include <math.h>
#include <stdio.h>
#include <stdlib.h>
#include <string.h>
#ifdef _OPENMP
#include <omp.h>
#endif

#define VOCAB 256
#define TOTAL_FREQ (1u << 24)
#define CDF_SCALE ((double)(TOTAL_FREQ - 256u))

static inline float u2f(uint32_t u) { float f; memcpy(&f, &u, 4); return f; }
static inline uint32_t f2u(float f) { uint32_t u; memcpy(&u, &f, 4); return u; }

/* bfloat16: the upper half of a float32, rounded to nearest even; NaN stays
 * a quiet NaN. */
uint16_t ref_f32_to_bf16(float x) {
    uint32_t u = f2u(x);
    if ((u & 0x7FFFFFFFu) > 0x7F800000u) return (uint16_t)((u >> 16) | 0x40u);
    return (uint16_t)((u + 0x7FFFu + ((u >> 16) & 1u)) >> 16);
}
float ref_bf16_to_f32(uint16_t h) { return u2f((uint32_t)h << 16); }
static inline float bf16r(float x) { return ref_bf16_to_f32(ref_f32_to_bf16(x)); }
static void bf16_round(float* p, size_t n) {
    for (size_t i = 0; i < n; ++i) p[i] = bf16r(p[i]);
}

/* =====================================================================
 * Math.  ref_expf/ref_logf are this project's own functions (the GPU
 * kernels evaluate the same operation sequence, so results agree bit for
 * bit).  ref_repro_exp/tanh/gelu restate the reference's software
 * activations (activations.hpp:33-117, device branch).
 * ===================================================================== */

/* exp(x): Cody-Waite reduction x = k*ln2 + r, |r| <= ln2/2, with ln2 split
 * into a float head and tail; e^r by its degree-7 Taylor polynomial in
 * Horner form (fused multiply-adds); 2^k assembled in the exponent field.
 * Inputs below -87 return 0 so every non-zero result is a normal float. */
static float exp_core(float x) {
    const float LOG2E = 1.44269504088896340736f;
    const float LN2_HI = 0.693147182464599609375f;
    const float LN2_LO = -1.904654323148236e-09f;
    float kf = rintf(x * LOG2E);
    float r = fmaf(-kf, LN2_HI, x);
    r = fmaf(-kf, LN2_LO, r);
    float p = 1.98412698412698412698e-4f;      /* 1/7! */
    p = fmaf(p, r, 1.38888888888888888889e-3f); /* 1/6! */
    p = fmaf(p, r, 8.33333333333333333333e-3f); /* 1/5! */
    p = fmaf(p, r, 4.16666666666666666667e-2f); /* 1/4! */
    p = fmaf(p, r, 1.66666666666666666667e-1f); /* 1/3! */
    p = fmaf(p, r, 0.5f);
    p = fmaf(p, r, 1.0f);
    p = fmaf(p, r, 1.0f);
    int k = (int)kf;
    if (k > 127) return (p * u2f((uint32_t)(127 + 127) << 23)) * 2.0f;
    return p * u2f((uint32_t)(k + 127) << 23);
}

float ref_expf(float x) {
    if (x != x) return x;
    if (x > 88.72283935546875f) return INFINITY;
    if (x < -87.0f) return 0.0f;
    return exp_core(x);
}

/* 2^t for t <= 0: the selective scan's decay exp(-exp(A_log) dt) in base
 * 2 (the layer holds na2 = -exp(A_log) * log2(e), ref_scan_na2, and the
 * scan takes 2^t of t = na2 * dt) and the CDF's exp(l - max) as
 * 2^((l - max) log2(e)).  t is clamped into [-126, 0] (fmaxf turns a
 * NaN into -126) and split as k + r, k = rint(t), r = t - k in [-1/2, 1/2]
 * (exact); 2^r is a degree-6 polynomial with 2^0 = 1 exact (coefficients
 * fitted to the relative error of 2^r on [-1/2, 1/2]) and 2^k is applied
 * with ldexpf, exact here.  The least result is 2^-126.  This is the exp
 * of the HIP scan and CDF kernels, operation for operation. */
float ref_exp2_neg(float t) {
    float s = fminf(fmaxf(t, -126.0f), 0.0f);
    float k = rintf(s);
    float r = s - k;
    float p = 0x1.41fbbap-13f;
    p = fmaf(p, r, 0x1.5f3e54p-10f);
    p = fmaf(p, r, 0x1.3b2d4cp-7f);
    p = fmaf(p, r, 0x1.c6aee8p-5f);
    p = fmaf(p, r, 0x1.ebfbdcp-3f);
    p = fmaf(p, r, 0x1.62e430p-1f);
    p = fmaf(p, r, 1.0f);
    return ldexpf(p, (int)k);
}

/* the scan's base-2 decay coefficient -exp(A_log) * log2(e) */
float ref_scan_na2(float a_log) { return -ref_expf(a_log) * 1.44269504088896340736f; }

/* log(y) for y > 0: y = 2^e * m with m in [sqrt(1/2), sqrt(2)],
 * log(m) = 2 atanh(s), s = (m-1)/(m+1), series to s^11. */
float ref_logf(float y) {
    if (y != y) return y;
    if (y == INFINITY) return y;
    if (y <= 0.0f) return (y == 0.0f) ? -INFINITY : NAN;
    uint32_t u = f2u(y);
    int e = (int)(u >> 23) - 127;
    if ((u >> 23) == 0) { /* subnormal: renormalise by 2^23 */
        y = y * 8388608.0f;
        u = f2u(y);
        e = (int)(u >> 23) - 127 - 23;
    }
    float m = u2f((u & 0x007FFFFFu) | 0x3F800000u);
    if (m > 1.41421353816986083984375f) { m = m * 0.5f; e += 1; }
    float s = (m - 1.0f) / (m + 1.0f);
    float s2 = s * s;
    float p = 0.0909090909090909090909f;        /* 1/11 */
    p = fmaf(p, s2, 0.111111111111111111111f);  /* 1/9 */
    p = fmaf(p, s2, 0.142857142857142857143f);  /* 1/7 */
    p = fmaf(p, s2, 0.2f);                      /* 1/5 */
    p = fmaf(p, s2, 0.333333333333333333333f);  /* 1/3 */
    float two_s = s + s;
    float lm = fmaf(two_s * s2, p, two_s);
    const float LN2_HI = 0.693147182464599609375f;
    const float LN2_LO = -1.904654323148236e-09f;
    float ef = (float)e;
    return fmaf(ef, LN2_HI, fmaf(ef, LN2_LO, lm));
}

/* activations.hpp:33-84 (GPU branch; __fadd_rn/__fmul_rn order kept). */
float ref_repro_exp(float x) {
    if (x <= -88.0f) return 0.0f;
    if (x >= 88.0f) x = 88.0f;
    float kf = floorf(x * 1.44269504088896340736f + 0.5f);
    int k = (int)kf;
    float r = x + (-(kf * 0.69314718055994530942f));
    float t = 0.008333333333f + r * 0.001388888889f;
    t = 0.041666666667f + r * t;
    t = 0.166666666667f + r * t;
    t = 0.5f + r * t;
    t = 1.0f + r * t;
    t = 1.0f + r * t;
    return t * u2f((uint32_t)((k + 127) << 23));
}

/* activations.hpp:87-98 */
float ref_repro_tanh(float x) {
    float ax = x < 0.0f ? -x : x;
    if (ax > 10.0f) return (x > 0.0f) ? 1.0f : -1.0f;
    float e2x = ref_repro_exp(2.0f * x);
    return (e2x + -1.0f) / (e2x + 1.0f);
}

/* activations.hpp:105-117, tanh-approximated GELU */
float ref_gelu(float x) {
    float cube = (x * x) * x;
    float inner = 0.79788456080286535588f * (x + 0.044715f * cube);
    float th = ref_repro_tanh(inner);
    return 0.5f * (x * (1.0f + th));
}

/* mamba_kernels.cu:188-189 / :140-141 form: v * (1 / (1 + exp(-v))) */
float ref_silu(float x) {
    float sg = 1.0f / (1.0f + ref_expf(-x));
    return x * sg;
}

/* inference_kernels.cu:376-382: unthresholded log(1 + exp(x)) */
float ref_softplus(float x) { return ref_logf(1.0f + ref_expf(x)); }

/* boa_gpu.hpp:16-43: IEEE half -> float widening */
float ref_half_to_float(uint16_t h) {
    uint32_t sign = (uint32_t)(h >> 15) << 31;
    uint32_t ex = (h >> 10) & 0x1Fu;
    uint32_t mant = h & 0x3FFu;
    uint32_t out;
    if (ex == 0) {
        if (mant == 0) {
            out = sign;
        } else {
            int e = 1;
            while (!(mant & 0x400u)) { mant <<= 1; e--; }
            mant &= 0x3FFu;
            out = sign | ((uint32_t)(127 - 15 + e) << 23) | (mant << 13);
        }
    } else if (ex == 31) {
        out = sign | 0x7F800000u | (mant << 13);
    } else {
        out = sign | ((ex - 15 + 127) << 23) | (mant << 13);
    }
    return u2f(out);
}

/* =====================================================================
 * Range coder (range_coder_kernels.cu:46-60 init, :934-964 encode step,
 * :279-313 finish, :319-335 decoder init, :572-627 decoder step).
 * ===================================================================== */
void ref_rc_enc_init(ref_rc_enc* st) {
    st->lower = 0;
    st->range = ~(uint64_t)0;
    st->inverted_num = 0;
    st->first_inv_lower_word = 0;
    st->write_idx_words = 0;
    st->pad_ = 0;
}

void ref_rc_enc_put(ref_rc_enc* st, uint32_t left, uint32_t prob, uint32_t* out) {
    if (prob == 0) prob = 1;
    uint64_t scale = st->range >> 24;
    uint64_t old_lower = st->lower;
    st->range = scale * (uint64_t)prob;
    st->lower = st->lower + scale * (uint64_t)left;
    if (st->inverted_num > 0) {
        uint64_t sum = st->lower + st->range;
        if (sum > st->lower) {
            int carry = st->lower < old_lower;
            uint32_t first = carry ? st->first_inv_lower_word + 1u : st->first_inv_lower_word;
            uint32_t rest = carry ? 0u : 0xFFFFFFFFu;
            out[st->write_idx_words++] = first;
            for (int k = 1; k < st->inverted_num; ++k) out[st->write_idx_words++] = rest;
            st->inverted_num = 0;
        }
    }
    /* one shift always suffices (range >= 2^8 after the update); bounded */
    for (int it = 0; it < 2 && st->range < ((uint64_t)1 << 32); ++it) {
        uint32_t lower_word = (uint32_t)(st->lower >> 32);
        st->lower <<= 32;
        st->range <<= 32;
        if (st->inverted_num > 0) {
            st->inverted_num++;
        } else {
            uint64_t sum = st->lower + st->range;
            if (sum > st->lower) {
                out[st->write_idx_words++] = lower_word;
            } else {
                st->inverted_num = 1;
                st->first_inv_lower_word = lower_word;
            }
        }
    }
}

int32_t ref_rc_enc_finish(ref_rc_enc* st, uint32_t* out) {
    if (st->range == ~(uint64_t)0) return 0;
    uint64_t point = st->lower + (((uint64_t)1 << 32) - 1);
    if (st->inverted_num > 0) {
        int carry = point < st->lower;
        uint32_t first = carry ? st->first_inv_lower_word + 1u : st->first_inv_lower_word;
        uint32_t rest = carry ? 0u : 0xFFFFFFFFu;
        out[st->write_idx_words++] = first;
        for (int k = 1; k < st->inverted_num; ++k) out[st->write_idx_words++] = rest;
        st->inverted_num = 0;
    }
    uint32_t point_word = (uint32_t)(point >> 32);
    out[st->write_idx_words++] = point_word;
    uint64_t upper = st->lower + st->range;
    if ((uint32_t)(upper >> 32) == point_word) out[st->write_idx_words++] = 0u;
    return st->write_idx_words;
}

void ref_rc_dec_init(ref_rc_dec* st, const uint32_t* in, int32_t n_words) {
    st->lower = 0;
    st->range = ~(uint64_t)0;
    st->point = 0;
    st->read_idx_words = 0;
    st->pad_ = 0;
    for (int k = 0; k < 2; ++k) {
        uint32_t w = (st->read_idx_words < n_words) ? in[st->read_idx_words++] : 0u;
        st->point = (st->point << 32) | (uint64_t)w;
    }
}

uint32_t ref_rc_dec_target(const ref_rc_dec* st) {
    uint64_t scale = st->range >> 24;
    uint64_t q = (st->point - st->lower) / scale;
    if (q >= TOTAL_FREQ) q = TOTAL_FREQ - 1;
    return (uint32_t)q;
}

void ref_rc_dec_advance(ref_rc_dec* st, uint32_t low, uint32_t high, const uint32_t* in,
                        int32_t n_words) {
    uint64_t scale = st->range >> 24;
    uint32_t prob = high - low;
    if (prob == 0) prob = 1;
    st->lower = st->lower + scale * (uint64_t)low;
    st->range = scale * (uint64_t)prob;
    for (int it = 0; it < 2 && st->range < ((uint64_t)1 << 32); ++it) {
        st->lower <<= 32;
        st->range <<= 32;
        uint32_t w = (st->read_idx_words < n_words) ? in[st->read_idx_words++] : 0u;
        st->point = (st->point << 32) | (uint64_t)w;
    }
}

int32_t ref_rc_encode_cdf_stream(const uint32_t* cdf, const uint8_t* syms, int32_t n_sym,
                                 uint32_t* out) {
    ref_rc_enc st;
    ref_rc_enc_init(&st);
    for (int32_t i = 0; i < n_sym; ++i) {
        const uint32_t* c = cdf + (size_t)i * 257;
        uint32_t s = syms[i];
        ref_rc_enc_put(&st, c[s], c[s + 1] - c[s], out);
    }
    return ref_rc_enc_finish(&st, out);
}

void ref_rc_decode_cdf_stream(const uint32_t* cdf, int32_t n_sym, const uint32_t* in,
                              int32_t n_words, uint8_t* syms_out) {
    ref_rc_dec st;
    ref_rc_dec_init(&st, in, n_words);
    for (int32_t i = 0; i < n_sym; ++i) {
        const uint32_t* c = cdf + (size_t)i * 257;
        uint32_t q = ref_rc_dec_target(&st);
        int s = 0;
        uint32_t lo = 0, hi = 0;
        for (int k = 0; k < VOCAB; ++k) {
            if (q >= c[k] && q < c[k + 1]) { s = k; lo = c[k]; hi = c[k + 1]; break; }
        }
        syms_out[i] = (uint8_t)s;
        ref_rc_dec_advance(&st, lo, hi, in, n_words);
    }
}

/* =====================================================================
 * Deterministic CDF (range_coder_kernels.cu:504-561 decoder, :856-913
 * encoder).  The reference runs one 32-lane warp per token: lane l owns
 * symbols 8l..8l+7; max by shuffle-down tree; per-lane sequential double
 * sum; total by warpReduceSumDouble (shuffle-down 16,8,4,2,1, lane 0's
 * value is used); exclusive lane prefix by warpScanSumDouble (Hillis-
 * Steele, offsets 1..16); then the lane-boundary monotonicity fix-up.
 * The exponentials e_j = exp((l_j - max) / T) (the reference's exp_fast)
 * are this project's 2^((l_j - max) / T * log2(e)) (ref_exp2_neg).
 * ===================================================================== */
static double tree_sum32(const double* v_in) {
    double v[32];
    memcpy(v, v_in, sizeof v);
    for (int off = 16; off > 0; off >>= 1)
        for (int i = 0; i < off; ++i) v[i] = v[i] + v[i + off];
    return v[0];
}

static void scan32_inclusive(const double* in, double* out) {
    double v[32], nv[32];
    memcpy(v, in, sizeof v);
    for (int off = 1; off <= 16; off <<= 1) {
        for (int i = 0; i < 32; ++i) nv[i] = (i >= off) ? v[i] + v[i - off] : v[i];
        memcpy(v, nv, sizeof v);
    }
    memcpy(out, v, sizeof v);
}

/* mode 0 (used everywhere): the lane-boundary fix-up propagates lane by
 * lane, lane l comparing against lane l-1's already fixed last value, so the
 * result is monotone.  mode 1: the reference's lock-step form, where every
 * lane reads its neighbour before any lane writes; when two adjacent lanes
 * both shift it can leave s_cdf[8l] < s_cdf[8l-1], a zero-frequency symbol
 * whose encoding the decoder cannot recover.  The two modes agree bit for
 * bit whenever mode 1's result is monotone. */
void ref_cdf_build_mode(const float* logits, const float* bias, float inv_temperature,
                        double* s_cdf, int32_t mode) {
    float vals[VOCAB];
    float lane_max[32];
    for (int l = 0; l < 32; ++l) {
        float m = -1e30f;
        for (int i = 0; i < 8; ++i) {
            int c = l * 8 + i;
            float v = bias ? logits[c] + bias[c] : logits[c];
            vals[c] = v;
            m = fmaxf(m, v);
        }
        lane_max[l] = m;
    }
    float mx = lane_max[0];
    for (int l = 1; l < 32; ++l) mx = fmaxf(mx, lane_max[l]);

    double lane_sum[32];
    for (int l = 0; l < 32; ++l) {
        double s = 0.0;
        for (int i = 0; i < 8; ++i) {
            int c = l * 8 + i;
            float e = ref_exp2_neg(((vals[c] - mx) * inv_temperature) * 1.44269504088896340736f);
            vals[c] = e;
            s += (double)e;
        }
        lane_sum[l] = s;
    }
    double total = tree_sum32(lane_sum);
    double inv = 1.0 / total;
    double ts[32], pre[32];
    for (int l = 0; l < 32; ++l) ts[l] = lane_sum[l] * inv;
    scan32_inclusive(ts, pre);
    for (int l = 0; l < 32; ++l) {
        double running = pre[l] - ts[l];
        for (int i = 0; i < 8; ++i) {
            s_cdf[l * 8 + i] = running;
            running += (double)vals[l * 8 + i] * inv;
        }
    }
    s_cdf[256] = 1.0;
    if (mode == 1) {
        double delta[32];
        int fix[32];
        fix[0] = 0;
        delta[0] = 0.0;
        for (int l = 1; l < 32; ++l) {
            double prev_end = s_cdf[l * 8 - 1];
            double my_start = s_cdf[l * 8];
            fix[l] = my_start < prev_end;
            delta[l] = fix[l] ? prev_end - my_start : 0.0;
        }
        for (int l = 1; l < 32; ++l)
            if (fix[l])
                for (int i = 0; i < 8; ++i) s_cdf[l * 8 + i] += delta[l];
    } else {
        for (int l = 1; l < 32; ++l) {
            double prev_end = s_cdf[l * 8 - 1];
            double my_start = s_cdf[l * 8];
            if (my_start < prev_end) {
                double delta = prev_end - my_start;
                for (int i = 0; i < 8; ++i) s_cdf[l * 8 + i] += delta;
            }
        }
    }
}

void ref_cdf_build(const float* logits, const float* bias, float inv_temperature,
                   double* s_cdf) {
    ref_cdf_build_mode(logits, bias, inv_temperature, s_cdf, 0);
}

static inline uint32_t q_low(const double* s_cdf, int k) {
    return (uint32_t)(s_cdf[k] * CDF_SCALE) + (uint32_t)k;
}
static inline uint32_t q_high(const double* s_cdf, int k) {
    if (k == 255) return TOTAL_FREQ;
    return (uint32_t)(s_cdf[k + 1] * CDF_SCALE) + (uint32_t)(k + 1);
}

void ref_cdf_interval(const double* s_cdf, int32_t k, uint32_t* low, uint32_t* high) {
    *low = q_low(s_cdf, k);
    *high = q_high(s_cdf, k);
}

/* gpu_range_coder.py:57-79 (build_cdf_fast, the Python GPU codec's CDF):
 * double sums in index order; a negative scaled running sum (impossible for
 * valid probabilities) is taken as 0. */
void ref_cdf_from_probs(const float* probs, int32_t K, uint32_t* cdf) {
    const uint32_t total = TOTAL_FREQ, free_w = total - (uint32_t)K;
    double norm = 0.0;
    for (int i = 0; i < K; ++i) norm += (double)probs[i];
    if (!(norm > 0.0) || !isfinite(norm)) {
        const uint32_t step = free_w / (uint32_t)K + 1u;
        uint32_t acc = 0;
        for (int i = 0; i < K; ++i) { cdf[i] = acc; acc += step; }
    } else {
        const double scale = (double)free_w / norm;
        double cum = 0.0;
        for (int i = 0; i < K; ++i) {
            const double v = cum * scale;
            cdf[i] = (uint32_t)(v > 0.0 ? v : 0.0) + (uint32_t)i;
            cum += (double)probs[i];
        }
    }
    cdf[K] = total;
}

void ref_cdf_quantize(const double* s_cdf, uint32_t* qcdf) {
    for (int k = 0; k < VOCAB; ++k) qcdf[k] = q_low(s_cdf, k);
    qcdf[256] = TOTAL_FREQ;
}

int32_t ref_cdf_search(const double* s_cdf, uint32_t target, uint32_t* low, uint32_t* high) {
    for (int k = 0; k < VOCAB; ++k) {
        uint32_t l = q_low(s_cdf, k), h = q_high(s_cdf, k);
        if (target >= l && target < h) { *low = l; *high = h; return k; }
    }
    *low = 0;
    *high = 0;
    return 0;
}

/* =====================================================================
 * Model (mambav1 only: x + FF(LN2(Mamba(LN1(x)))), head Linear-ReLU-Linear)
 * Weights are kept like the reference keeps them on the device: Linear
 * weights transposed to [in][out] (boa_gpu.hpp:46-54, 213-222).
 * ===================================================================== */
typedef struct {
    float *ln1_w, *ln1_b;
    float *w_in, *b_in;      /* [d][2di], [2di] */
    float *conv_w, *conv_b;  /* [di][4], [di] */
    float *w_x;              /* [di][R], R = r + 2 ds */
    float *w_dt, *b_dt;      /* [r][di], [di] */
    float *a_log, *dd;       /* [di][ds], [di] */
    float *w_out, *b_out;    /* [di][d], [d] */
    float *ln2_w, *ln2_b;
    float *w1, *b1;          /* [d][4d], [4d] */
    float *w2, *b2;          /* [4d][d], [d] */
    float *na2;              /* -exp(A_log) log2(e), [di][ds] (mamba_kernels.cu:430-437) */
} ref_layer;

struct ref_model {
    int d, L, di, r, ds, dc, R;
    int bf16;                /* 1: bf16 weights and activations (ref_model_set_bf16) */
    float* emb;              /* [256][d] */
    ref_layer* layers;
    float *hw1, *hb1;        /* [d][d], [d] */
    float *hw2, *hb2;        /* [d][256], [256] */
};

struct ref_state {
    int lanes;
    int d, L, di, ds, dc;
    float* conv;             /* [L][lanes][di][dc] */
    float* ssm;              /* [L][lanes][di][ds] */
};

int64_t ref_model_expected_bytes(int32_t d, int32_t L, int32_t ds, int32_t fp16) {
    int64_t di = 2 * (int64_t)d, r = (d + 15) / 16, R = r + 2 * (int64_t)ds;
    int64_t per_layer = 2 * d + 2 * di * d + 2 * di + di * 4 + di + R * di + di * r + di +
                        di * ds + di + d * di + d + 2 * d + 4 * (int64_t)d * d + 4 * d +
                        4 * (int64_t)d * d + d;
    int64_t elems = 256 * (int64_t)d + L * per_layer + (int64_t)d * d + d + 256 * (int64_t)d + 256;
    return 4 + elems * (fp16 ? 2 : 4);
}

typedef struct {
    const uint8_t* p;
    int64_t n, pos;
    int fp16;
    int bad;
} wreader;

static void rd_vec(wreader* r, float* dst, int64_t count) {
    int64_t esz = r->fp16 ? 2 : 4;
    if (r->bad || r->pos + count * esz > r->n) { r->bad = 1; return; }
    if (r->fp16) {
        for (int64_t i = 0; i < count; ++i) {
            uint16_t h;
            memcpy(&h, r->p + r->pos + 2 * i, 2);
            dst[i] = ref_half_to_float(h);
        }
    } else {
        memcpy(dst, r->p + r->pos, (size_t)(count * 4));
    }
    r->pos += count * esz;
}

/* read a PyTorch [rows][cols] Linear weight and store it as [cols][rows] */
static void rd_linear_t(wreader* r, float* dst, int rows, int cols) {
    float* tmp = (float*)malloc(sizeof(float) * (size_t)rows * cols);
    rd_vec(r, tmp, (int64_t)rows * cols);
    for (int i = 0; i < rows; ++i)
        for (int j = 0; j < cols; ++j) dst[(size_t)j * rows + i] = tmp[(size_t)i * cols + j];
    free(tmp);
}

static float* fa(size_t n) { return (float*)calloc(n ? n : 1, sizeof(float)); }

ref_model* ref_model_load(const char* path, int32_t d, int32_t L, int32_t ds, char* err,
                          int32_t err_len) {
    FILE* f = fopen(path, "rb");
    if (!f) { snprintf(err, err_len, "cannot open %s", path); return NULL; }
    fseek(f, 0, SEEK_END);
    long n = ftell(f);
    fseek(f, 0, SEEK_SET);
    uint8_t* buf = (uint8_t*)malloc((size_t)n + 1);
    if (fread(buf, 1, (size_t)n, f) != (size_t)n) {
        fclose(f); free(buf);
        snprintf(err, err_len, "read error"); return NULL;
    }
    fclose(f);
    wreader rd = {buf, n, 0, 0, 0};
    /* boa_gpu.hpp:994-1006: "BOA" + 0x01 -> fp16, other 4th byte -> fp32,
     * no "BOA" -> headerless fp32 */
    int has_hdr = n >= 4 && buf[0] == 'B' && buf[1] == 'O' && buf[2] == 'A';
    if (has_hdr) { rd.fp16 = buf[3] == 0x01; rd.pos = 4; }
    int64_t expect = ref_model_expected_bytes(d, L, ds, rd.fp16) - (has_hdr ? 0 : 4);
    if (n != expect) {
        snprintf(err, err_len, "weight file has %ld bytes, expected %lld for d_model=%d n_layers=%d d_state=%d",
                 n, (long long)expect, d, L, ds);
        free(buf); return NULL;
    }
    ref_model* m = (ref_model*)calloc(1, sizeof(ref_model));
    m->d = d; m->L = L; m->di = 2 * d; m->r = (d + 15) / 16; m->ds = ds; m->dc = 4;
    m->R = m->r + 2 * ds;
    int di = m->di, r = m->r, R = m->R;
    m->emb = fa((size_t)256 * d);
    rd_vec(&rd, m->emb, (int64_t)256 * d);
    m->layers = (ref_layer*)calloc((size_t)L, sizeof(ref_layer));
    for (int l = 0; l < L; ++l) {
        ref_layer* y = &m->layers[l];
        y->ln1_w = fa(d); y->ln1_b = fa(d);
        rd_vec(&rd, y->ln1_w, d); rd_vec(&rd, y->ln1_b, d);
        y->w_in = fa((size_t)d * 2 * di); y->b_in = fa(2 * di);
        rd_linear_t(&rd, y->w_in, 2 * di, d); rd_vec(&rd, y->b_in, 2 * di);
        y->conv_w = fa((size_t)di * 4); y->conv_b = fa(di);
        rd_vec(&rd, y->conv_w, (int64_t)di * 4); rd_vec(&rd, y->conv_b, di);
        y->w_x = fa((size_t)di * R);
        rd_linear_t(&rd, y->w_x, R, di);
        y->w_dt = fa((size_t)r * di); y->b_dt = fa(di);
        rd_linear_t(&rd, y->w_dt, di, r); rd_vec(&rd, y->b_dt, di);
        y->a_log = fa((size_t)di * ds); y->dd = fa(di);
        rd_vec(&rd, y->a_log, (int64_t)di * ds); rd_vec(&rd, y->dd, di);
        y->w_out = fa((size_t)di * d); y->b_out = fa(d);
        rd_linear_t(&rd, y->w_out, d, di); rd_vec(&rd, y->b_out, d);
        y->ln2_w = fa(d); y->ln2_b = fa(d);
        rd_vec(&rd, y->ln2_w, d); rd_vec(&rd, y->ln2_b, d);
        y->w1 = fa((size_t)d * 4 * d); y->b1 = fa(4 * d);
        rd_linear_t(&rd, y->w1, 4 * d, d); rd_vec(&rd, y->b1, 4 * d);
        y->w2 = fa((size_t)4 * d * d); y->b2 = fa(d);
        rd_linear_t(&rd, y->w2, d, 4 * d); rd_vec(&rd, y->b2, d);
        y->na2 = fa((size_t)di * ds);
        for (int i = 0; i < di * ds; ++i) y->na2[i] = ref_scan_na2(y->a_log[i]);
    }
    m->hw1 = fa((size_t)d * d); m->hb1 = fa(d);
    rd_linear_t(&rd, m->hw1, d, d); rd_vec(&rd, m->hb1, d);
    m->hw2 = fa((size_t)d * 256); m->hb2 = fa(256);
    rd_linear_t(&rd, m->hw2, 256, d); rd_vec(&rd, m->hb2, 256);
    free(buf);
    if (rd.bad || rd.pos != n) {
        snprintf(err, err_len, "weight file truncated");
        ref_model_free(m);
        return NULL;
    }
    return m;
}

void ref_model_free(ref_model* m) {
    if (!m) return;
    for (int l = 0; l < m->L; ++l) {
        ref_layer* y = &m->layers[l];
        float* ps[] = {y->ln1_w, y->ln1_b, y->w_in, y->b_in, y->conv_w, y->conv_b, y->w_x,
                       y->w_dt, y->b_dt, y->a_log, y->dd, y->w_out, y->b_out, y->ln2_w,
                       y->ln2_b, y->w1, y->b1, y->w2, y->b2, y->na2};
        for (size_t i = 0; i < sizeof ps / sizeof ps[0]; ++i) free(ps[i]);
    }
    free(m->layers);
    free(m->emb); free(m->hw1); free(m->hb1); free(m->hw2); free(m->hb2);
    free(m);
}

int32_t ref_model_set_bf16(ref_model* m) {
    if (!m || m->bf16) return m ? 0 : -1;
    int d = m->d, di = m->di, R = m->R;
    for (int l = 0; l < m->L; ++l) {
        ref_layer* y = &m->layers[l];
        bf16_round(y->w_in, (size_t)d * 2 * di);
        bf16_round(y->w_x, (size_t)di * R);
        bf16_round(y->w_out, (size_t)di * d);
        bf16_round(y->w1, (size_t)d * 4 * d);
        bf16_round(y->w2, (size_t)4 * d * d);
    }
    bf16_round(m->hw1, (size_t)d * d);
    bf16_round(m->hw2, (size_t)d * 256);
    m->bf16 = 1;
    return 0;
}

ref_state* ref_state_new(const ref_model* m, int32_t lanes) {
    ref_state* s = (ref_state*)calloc(1, sizeof(ref_state));
    s->lanes = lanes; s->d = m->d; s->L = m->L; s->di = m->di; s->ds = m->ds; s->dc = m->dc;
    s->conv = fa((size_t)m->L * lanes * m->di * m->dc);
    s->ssm = fa((size_t)m->L * lanes * m->di * m->ds);
    return s;
}
void ref_state_reset(ref_state* s) {
    memset(s->conv, 0, sizeof(float) * (size_t)s->L * s->lanes * s->di * s->dc);
    memset(s->ssm, 0, sizeof(float) * (size_t)s->L * s->lanes * s->di * s->ds);
}
void ref_state_free(ref_state* s) {
    if (!s) return;
    free(s->conv); free(s->ssm); free(s);
}
static inline float* conv_state(const ref_state* s, int l, int lane) {
    return s->conv + ((size_t)l * s->lanes + lane) * s->di * s->dc;
}
static inline float* ssm_state(const ref_state* s, int l, int lane) {
    return s->ssm + ((size_t)l * s->lanes + lane) * s->di * s->ds;
}

/* ---- GEMM: C[M][N] = act(A[M][K] (lda) * W[K][N] + bias) + residual.
 * Each output is a K-ordered fused multiply-add chain starting from 0
 * (gemm_kernels.cu:283-295), then `acc + bias` (0 when absent, :306),
 * then the activation (:307-309), then `+ residual` (:310). */
enum { ACT_NONE = 0, ACT_GELU = 1, ACT_RELU = 2 };

static void gemm_rows(const float* A, int lda, const float* W, int K, int N, const float* bias,
                      int act, const float* res, int ldr, float* C, int ldc, int M) {
    enum { RB = 4, JB = 256 };
    float acc[RB][JB];
    for (int m0 = 0; m0 < M; m0 += RB) {
        int mr = M - m0 < RB ? M - m0 : RB;
        for (int j0 = 0; j0 < N; j0 += JB) {
            int nj = N - j0 < JB ? N - j0 : JB;
            for (int i = 0; i < mr; ++i)
                for (int j = 0; j < nj; ++j) acc[i][j] = 0.0f;
            for (int k = 0; k < K; ++k) {
                const float* w = W + (size_t)k * N + j0;
                for (int i = 0; i < mr; ++i) {
                    float a = A[(size_t)(m0 + i) * lda + k];
                    float* ac = acc[i];
                    for (int j = 0; j < nj; ++j) ac[j] = fmaf(a, w[j], ac[j]);
                }
            }
            for (int i = 0; i < mr; ++i) {
                float* c = C + (size_t)(m0 + i) * ldc + j0;
                for (int j = 0; j < nj; ++j) {
                    float v = acc[i][j] + (bias ? bias[j0 + j] : 0.0f);
                    if (act == ACT_GELU) v = ref_gelu(v);
                    else if (act == ACT_RELU) v = fmaxf(0.0f, v);
                    if (res) v = v + res[(size_t)(m0 + i) * ldr + j0 + j];
                    c[j] = v;
                }
            }
        }
    }
}

/* LN1 (inference_kernels.cu:293-348): lane l of a 32-lane warp sums
 * elements l, l+32, ... sequentially; lanes combine by shuffle-down tree. */
static void layernorm_warp_row(const float* x, const float* w, const float* b, float* out, int N) {
    float ls[32], lq[32];
    int per = (N + 31) / 32;
    for (int l = 0; l < 32; ++l) {
        float s = 0.0f, q = 0.0f;
        for (int e = 0; e < per; ++e) {
            int idx = l + e * 32;
            if (idx < N) { float v = x[idx]; s = s + v; q = q + v * v; }
        }
        ls[l] = s; lq[l] = q;
    }
    for (int off = 16; off > 0; off >>= 1)
        for (int i = 0; i < off; ++i) { ls[i] = ls[i] + ls[i + off]; lq[i] = lq[i] + lq[i + off]; }
    float mean = ls[0] / (float)N;
    float var = lq[0] / (float)N - mean * mean;
    float inv_std = 1.0f / sqrtf(var + 1e-5f);
    for (int i = 0; i < N; ++i) out[i] = ((x[i] - mean) * inv_std) * w[i] + b[i];
}

/* LN2 (inference_kernels.cu:229-277): one thread per row, sequential sums */
static void layernorm_seq_row(const float* x, const float* w, const float* b, float* out, int N) {
    float s = 0.0f, q = 0.0f;
    for (int i = 0; i < N; ++i) { float v = x[i]; s = s + v; q = q + v * v; }
    float mean = s / (float)N;
    float var = q / (float)N - mean * mean;
    float inv_std = 1.0f / sqrtf(var + 1e-5f);
    for (int i = 0; i < N; ++i) out[i] = ((x[i] - mean) * inv_std) * w[i] + b[i];
}

typedef struct {
    float *x, *xn, *xz, *cv, *delta, *y, *hid, *hh;
    int cap;
} scratch_t;

static void scratch_init(scratch_t* s, const ref_model* m, int rows) {
    int d = m->d, di = m->di;
    s->cap = rows;
    s->x = fa((size_t)rows * d);
    s->xn = fa((size_t)rows * d);
    s->xz = fa((size_t)rows * 2 * di);
    s->cv = fa((size_t)rows * di);
    s->delta = fa((size_t)rows * m->R);
    s->y = fa((size_t)rows * di);
    s->hid = fa((size_t)rows * 4 * d);
    s->hh = fa((size_t)rows * d);
}
static void scratch_free(scratch_t* s) {
    free(s->x); free(s->xn); free(s->xz); free(s->cv); free(s->delta); free(s->y);
    free(s->hid); free(s->hh);
}

/* dt_proj + softplus + selective scan + D + SiLU(z) gate for one channel
 * d and one row, state h[ds] (mamba_kernels.cu:285-350 / :414-470 with
 * the dt_proj GEMM of boa_gpu.hpp:317-318 and the gate of :326). */
static inline float scan_row(const ref_layer* Ly, const ref_model* m, int dch, const float* delta_row,
                             float u, float z, float* h) {
    int r = m->r, ds = m->ds, di = m->di;
    float acc = 0.0f;
    for (int j = 0; j < r; ++j) acc = fmaf(delta_row[j], Ly->w_dt[(size_t)j * di + dch], acc);
    float dt = ref_softplus(acc + Ly->b_dt[dch]);
    const float* Bv = delta_row + r;
    const float* Cv = delta_row + r + ds;
    const float* na = Ly->na2 + (size_t)dch * ds;
    /* the reference's unfused update, every product and sum rounded on its
     * own (__fmul_rn / __fadd_rn at mamba_kernels.cu:332-335 and :453-461):
     * dB = dt B_n; h_n = (dA h_n) + (dB u); y = y + (h_n C_n) */
    float y = 0.0f;
    for (int n = 0; n < ds; ++n) {
        float dA = ref_exp2_neg(na[n] * dt);
        float dB = dt * Bv[n];
        h[n] = dA * h[n] + dB * u;
        y = y + h[n] * Cv[n];
    }
    y = y + Ly->dd[dch] * u;
    float sg = 1.0f / (1.0f + ref_expf(-z));
    return y * (z * sg);
}

/* scan_row over T consecutive tokens of one channel (dt_proj row w_dt[r],
 * its bias, D, the channel's A_log[ds] and state h[ds]; delta rows of
 * r + 2 ds floats): the chunk-mode scan of mamba_kernels.cu:414-470 with
 * the dt_proj + softplus of boa_gpu.hpp:317-318 and the gate of
 * mamba_kernels.cu:130-151.  A test hook for the update's rounding. */
void ref_scan_channel(const float* w_dt, float b_dt, float dd, const float* a_log, int32_t r,
                      int32_t ds, int32_t T, const float* delta, const float* u, const float* z,
                      float* h, float* y) {
    ref_layer Ly;
    ref_model m;
    float na2[64];
    memset(&Ly, 0, sizeof Ly);
    memset(&m, 0, sizeof m);
    for (int n = 0; n < ds && n < 64; ++n) na2[n] = ref_scan_na2(a_log[n]);
    Ly.w_dt = (float*)w_dt;  /* di = 1: w_dt[j * di + 0] = w_dt[j] */
    Ly.b_dt = &b_dt;
    Ly.dd = &dd;
    Ly.na2 = na2;
    m.r = r; m.ds = ds; m.di = 1; m.R = r + 2 * ds;
    for (int t = 0; t < T; ++t)
        y[t] = scan_row(&Ly, &m, 0, delta + (size_t)t * m.R, u[t], z[t], h);
}

/* One mambav1 block over `rows` rows held in sc->x.  chunk mode: the rows
 * are consecutive tokens of one lane (state index `lane`); step mode: row
 * i is lane lane0+i, one token each. */
static void block_rows(const ref_model* m, const ref_state* st, int l, scratch_t* sc, int rows,
                       int chunk_mode, int lane0) {
    const ref_layer* Ly = &m->layers[l];
    int d = m->d, di = m->di, R = m->R, ds = m->ds;
    const int bf = m->bf16;  /* bf16 mode: round every stored activation but x */
    for (int i = 0; i < rows; ++i)
        layernorm_warp_row(sc->x + (size_t)i * d, Ly->ln1_w, Ly->ln1_b, sc->xn + (size_t)i * d, d);
    if (bf) bf16_round(sc->xn, (size_t)rows * d);
    gemm_rows(sc->xn, d, Ly->w_in, d, 2 * di, Ly->b_in, ACT_NONE, NULL, 0, sc->xz, 2 * di, rows);
    if (bf) bf16_round(sc->xz, (size_t)rows * 2 * di);
    /* causal depthwise conv1d + SiLU */
    if (chunk_mode) {
        float* cs_all = conv_state(st, l, lane0);
        for (int c = 0; c < di; ++c) {
            float* cs = cs_all + (size_t)c * 4;
            const float* w = Ly->conv_w + (size_t)c * 4;
            for (int t = 0; t < rows; ++t) {
                float v = Ly->conv_b[c];
                for (int k = 0; k < 4; ++k) {
                    int te = t - 3 + k;
                    float xv = te >= 0 ? sc->xz[(size_t)te * 2 * di + c] : cs[4 + te];
                    v = v + xv * w[k];
                }
                sc->cv[(size_t)t * di + c] = ref_silu(v);
            }
            float nw[4];
            for (int k = 0; k < 4; ++k) {
                int te = rows - 4 + k;
                nw[k] = te >= 0 ? sc->xz[(size_t)te * 2 * di + c] : cs[4 + te];
            }
            memcpy(cs, nw, sizeof nw);
        }
    } else {
        for (int i = 0; i < rows; ++i) {
            float* cs_all = conv_state(st, l, lane0 + i);
            for (int c = 0; c < di; ++c) {
                float* s = cs_all + (size_t)c * 4;
                const float* w = Ly->conv_w + (size_t)c * 4;
                s[0] = s[1]; s[1] = s[2]; s[2] = s[3];
                s[3] = sc->xz[(size_t)i * 2 * di + c];
                float v = Ly->conv_b[c];
                for (int k = 0; k < 4; ++k) v = v + s[k] * w[k];
                sc->cv[(size_t)i * di + c] = ref_silu(v);
            }
        }
    }
    if (bf) bf16_round(sc->cv, (size_t)rows * di);
    gemm_rows(sc->cv, di, Ly->w_x, di, R, NULL, ACT_NONE, NULL, 0, sc->delta, R, rows);
    if (bf) bf16_round(sc->delta, (size_t)rows * R);
    if (chunk_mode) {
        float* hs = ssm_state(st, l, lane0);
        for (int c = 0; c < di; ++c) {
            float* h = hs + (size_t)c * ds;
            for (int t = 0; t < rows; ++t)
                sc->y[(size_t)t * di + c] = scan_row(Ly, m, c, sc->delta + (size_t)t * R,
                                                     sc->cv[(size_t)t * di + c],
                                                     sc->xz[(size_t)t * 2 * di + di + c], h);
        }
    } else {
        for (int i = 0; i < rows; ++i) {
            float* hs = ssm_state(st, l, lane0 + i);
            for (int c = 0; c < di; ++c)
                sc->y[(size_t)i * di + c] = scan_row(Ly, m, c, sc->delta + (size_t)i * R,
                                                     sc->cv[(size_t)i * di + c],
                                                     sc->xz[(size_t)i * 2 * di + di + c],
                                                     hs + (size_t)c * ds);
        }
    }
    /* out_proj, LN2, FF1+GELU, FF2+bias+residual(saved pre-LN1 x) */
    if (bf) bf16_round(sc->y, (size_t)rows * di);
    gemm_rows(sc->y, di, Ly->w_out, di, d, Ly->b_out, ACT_NONE, NULL, 0, sc->xn, d, rows);
    if (bf) bf16_round(sc->xn, (size_t)rows * d);
    for (int i = 0; i < rows; ++i)
        layernorm_seq_row(sc->xn + (size_t)i * d, Ly->ln2_w, Ly->ln2_b, sc->xn + (size_t)i * d, d);
    if (bf) bf16_round(sc->xn, (size_t)rows * d);
    gemm_rows(sc->xn, d, Ly->w1, d, 4 * d, Ly->b1, ACT_GELU, NULL, 0, sc->hid, 4 * d, rows);
    if (bf) bf16_round(sc->hid, (size_t)rows * 4 * d);
    gemm_rows(sc->hid, 4 * d, Ly->w2, 4 * d, d, Ly->b2, ACT_NONE, sc->x, d, sc->x, d, rows);
}

static void head_rows(const ref_model* m, scratch_t* sc, int rows, int add_bias, float* logits) {
    int d = m->d;
    const float* xin = sc->x;
    if (m->bf16) {  /* the residual stream stays fp32; head1 reads its bf16 copy */
        memcpy(sc->xn, sc->x, sizeof(float) * (size_t)rows * d);
        bf16_round(sc->xn, (size_t)rows * d);
        xin = sc->xn;
    }
    gemm_rows(xin, d, m->hw1, d, d, m->hb1, ACT_RELU, NULL, 0, sc->hh, d, rows);
    if (m->bf16) bf16_round(sc->hh, (size_t)rows * d);
    gemm_rows(sc->hh, d, m->hw2, d, 256, add_bias ? m->hb2 : NULL, ACT_NONE, NULL, 0, logits, 256, rows);
}

static void embed_rows(const ref_model* m, const uint8_t* tok, int rows, float* x) {
    for (int i = 0; i < rows; ++i)
        memcpy(x + (size_t)i * m->d, m->emb + (size_t)tok[i] * m->d, sizeof(float) * m->d);
}

static void forward_lane(const ref_model* m, ref_state* s, int lane, const uint8_t* tok, int T,
                         float* logits, scratch_t* sc) {
    for (int t0 = 0; t0 < T; t0 += sc->cap) {
        int n = T - t0 < sc->cap ? T - t0 : sc->cap;
        embed_rows(m, tok + t0, n, sc->x);
        for (int l = 0; l < m->L; ++l) block_rows(m, s, l, sc, n, 1, lane);
        head_rows(m, sc, n, 1, logits + (size_t)t0 * 256);
    }
}

static int pick_threads(int n_threads) {
#ifdef _OPENMP
    return n_threads > 0 ? n_threads : omp_get_max_threads();
#else
    (void)n_threads;
    return 1;
#endif
}

void ref_forward_chunk(const ref_model* m, ref_state* s, const uint8_t* tokens, int32_t lanes,
                       int32_t T, float* logits, int32_t n_threads) {
    int nt = pick_threads(n_threads);
#pragma omp parallel num_threads(nt)
    {
        scratch_t sc;
        scratch_init(&sc, m, 64);
#pragma omp for schedule(dynamic, 1)
        for (int b = 0; b < lanes; ++b)
            forward_lane(m, s, b, tokens + (size_t)b * T, T, logits + (size_t)b * T * 256, &sc);
        scratch_free(&sc);
    }
}

void ref_step(const ref_model* m, ref_state* s, const uint8_t* tokens, int32_t lanes,
              float* logits, int32_t add_bias, int32_t n_threads) {
    enum { G = 8 };
    int nt = pick_threads(n_threads);
    int groups = (lanes + G - 1) / G;
#pragma omp parallel num_threads(nt)
    {
        scratch_t sc;
        scratch_init(&sc, m, G);
#pragma omp for schedule(dynamic, 1)
        for (int g = 0; g < groups; ++g) {
            int b0 = g * G, n = lanes - b0 < G ? lanes - b0 : G;
            embed_rows(m, tokens + b0, n, sc.x);
            for (int l = 0; l < m->L; ++l) block_rows(m, s, l, &sc, n, 0, b0);
            head_rows(m, &sc, n, add_bias, logits + (size_t)b0 * 256);
        }
        scratch_free(&sc);
    }
}

/* =====================================================================
 * Container (boa.cpp:85-107 CRC-32, :158-176 LEB128, :190-277 reader,
 * :538-581 writer).
 * ===================================================================== */
uint32_t ref_crc32(const uint8_t* data, int64_t n) {
    uint32_t table[256];
    for (uint32_t i = 0; i < 256; ++i) {
        uint32_t c = i;
        for (int k = 0; k < 8; ++k) c = (c & 1) ? (0xEDB88320u ^ (c >> 1)) : (c >> 1);
        table[i] = c;
    }
    uint32_t c = 0xFFFFFFFFu;
    for (int64_t i = 0; i < n; ++i) c = table[(c ^ data[i]) & 0xFFu] ^ (c >> 8);
    return c ^ 0xFFFFFFFFu;
}

int32_t ref_uvarint_encode(uint64_t x, uint8_t* out) {
    int n = 0;
    for (;;) {
        uint8_t b = (uint8_t)(x & 0x7Fu);
        x >>= 7;
        out[n++] = (uint8_t)(b | (x ? 0x80u : 0u));
        if (!x) break;
    }
    return n;
}

static int uvarint_decode(const uint8_t* buf, int64_t end, int64_t* pos, uint64_t* out) {
    uint64_t x = 0;
    int shift = 0;
    for (;;) {
        if (*pos >= end || shift > 63) return -1;
        uint8_t b = buf[(*pos)++];
        x |= (uint64_t)(b & 0x7Fu) << shift;
        if (!(b & 0x80u)) break;
        shift += 7;
    }
    *out = x;
    return 0;
}

static uint32_t rd32(const uint8_t* p) { uint32_t v; memcpy(&v, p, 4); return v; }

int32_t ref_boa2_parse(const uint8_t* buf, int64_t n, ref_boa2_info* info, uint8_t* first_bytes,
                       uint64_t* offsets, uint64_t* lengths) {
    if (n < 32) return -1;
    if (memcmp(buf, "BOA2", 4) != 0) return -2;
    if (rd32(buf + 4) != 1) return -3;
    info->flags = rd32(buf + 8);
    memcpy(&info->total_size, buf + 12, 8);
    info->chunk_len = rd32(buf + 20);
    info->n_chunks = rd32(buf + 24);
    info->last_chunk_len = rd32(buf + 28);
    if (n < 33) return -1;
    uint8_t fp_len = buf[32];
    int64_t p = 33;
    info->interleave_batch = 0;
    if ((info->flags & 1u) && fp_len >= 4 && p + 4 <= n) info->interleave_batch = rd32(buf + p);
    p += fp_len;
    info->payload_off = p;
    int64_t idx = -1;
    int ver = 0;
    for (int64_t i = n - 4; i-- > 0;) {
        if (buf[i] == 'I' && buf[i + 1] == 'D' && buf[i + 2] == 'X') {
            if (buf[i + 3] == '2') { idx = i; ver = 2; break; }
            if (buf[i + 3] == '1') { idx = i; ver = 1; break; }
        }
    }
    if (idx < 0) return -4;
    if (n < idx + 8) return -5;
    if (rd32(buf + n - 4) != ref_crc32(buf + idx, n - idx - 4)) return -6;
    info->idx_off = idx;
    info->idx_version = ver;
    if (!first_bytes) return 0;
    int64_t q = idx + 4, end = n - 4;
    uint32_t nc = info->n_chunks;
    if (q + nc > end) return -7;
    for (uint32_t i = 0; i < nc; ++i) first_bytes[i] = buf[q++];
    if (ver == 1) {
        uint64_t prev = 0, dlt;
        for (uint32_t i = 0; i < nc; ++i) {
            if (uvarint_decode(buf, end, &q, &dlt)) return -7;
            prev += dlt;
            offsets[i] = prev;
        }
        for (uint32_t i = 0; i < nc; ++i)
            if (uvarint_decode(buf, end, &q, &lengths[i])) return -7;
    } else {
        uint64_t off = 0;
        for (uint32_t i = 0; i < nc; ++i) {
            if (uvarint_decode(buf, end, &q, &lengths[i])) return -7;
            offsets[i] = off;
            off += lengths[i];
        }
    }
    uint64_t payload = (uint64_t)(idx - info->payload_off);
    for (uint32_t i = 0; i < nc; ++i)
        if (offsets[i] + lengths[i] > payload) return -8;
    return 0;
}

/* =====================================================================
 * End-to-end compress / decompress (boa.cpp:280-582, :584-817).
 * Without warm-start lanes are independent, so every chunk is encoded on
 * its own: tiling and batching do not change a single bit of the output.
 * With warm-start (boa.cpp:310-319, 395-435) the B = min(gpu_batch, n)
 * lanes each run S = ceil(n / B) chunks in a row, lane b taking chunks
 * b*S + i, and the recurrent state carries from one chunk to the next:
 * compress forwards every byte of a chunk (boa.cpp:441-469 walks tiles up
 * to chunk_size), so the state that starts chunk b*S + i + 1 has consumed
 * all of chunk b*S + i.  The decoder here consumes the chunk's last byte
 * with one more step before the next chunk, which keeps it in step with
 * that compressor (boa.cpp:717-740 stops after chunk_size - 1 steps).
 * ===================================================================== */
void ref_free(void* p) { free(p); }

static int64_t pitch_words_for(int64_t chunk) { return (chunk * 10 + 4096 + 3) / 4; }

/* Codes bytes 1..len-1 of one chunk with the state in lane 0 of `s`
 * (boa.cpp:441-469 with range_coder_kernels.cu:854-858).  feed_all also
 * forwards the last byte so the state ends having consumed the whole chunk
 * (warm-start). */
static int32_t encode_with_state(const ref_model* m, ref_state* s, const uint8_t* chunk,
                                 int32_t len, int32_t tile, float temperature, uint32_t* words,
                                 int32_t cap_words, int feed_all) {
    int n_fwd = feed_all ? len : len - 1; /* positions forwarded */
    if (n_fwd <= 0) return 0;
    int T = tile > 0 ? tile : 256;
    if (T > 256) T = 256;
    scratch_t sc;
    scratch_init(&sc, m, T);
    float* logits = (float*)malloc(sizeof(float) * (size_t)T * 256);
    ref_rc_enc st;
    ref_rc_enc_init(&st);
    float inv_t = 1.0f / temperature;
    double s_cdf[257];
    int n_pos = len - 1; /* positions whose prediction is coded */
    for (int t0 = 0; t0 < n_fwd; t0 += T) {
        int n = n_fwd - t0 < T ? n_fwd - t0 : T;
        forward_lane(m, s, 0, chunk + t0, n, logits, &sc);
        for (int i = 0; i < n && t0 + i < n_pos; ++i) {
            ref_cdf_build(logits + (size_t)i * 256, NULL, inv_t, s_cdf);
            uint32_t lo, hi;
            ref_cdf_interval(s_cdf, chunk[t0 + i + 1], &lo, &hi);
            ref_rc_enc_put(&st, lo, hi - lo, words);
            if (st.write_idx_words > cap_words - 16) { /* cannot happen below 3 B/symbol */
                free(logits); scratch_free(&sc);
                return -1;
            }
        }
    }
    int32_t nw = n_pos > 0 ? ref_rc_enc_finish(&st, words) : 0;
    free(logits);
    scratch_free(&sc);
    return nw;
}

int32_t ref_encode_chunk(const ref_model* m, const uint8_t* chunk, int32_t len, int32_t tile,
                         float temperature, uint32_t* words, int32_t cap_words) {
    if (len <= 1) return 0;
    ref_state* s = ref_state_new(m, 1);
    int32_t nw = encode_with_state(m, s, chunk, len, tile, temperature, words, cap_words, 0);
    ref_state_free(s);
    return nw;
}

int32_t ref_compress(const ref_model* m, const uint8_t* data, int64_t n, const ref_codec_opts* o,
                     uint8_t** out, int64_t* out_len) {
    int64_t chunk = o->chunk_size > 0 ? o->chunk_size : 4096;
    int64_t nc64 = (n + chunk - 1) / chunk;
    if (o->max_chunks > 0 && nc64 > o->max_chunks) nc64 = o->max_chunks;
    int nc = (int)nc64;
    int64_t processed = n < nc64 * chunk ? n : nc64 * chunk;
    int64_t last_len = nc > 1 ? processed - (int64_t)(nc - 1) * chunk : processed;
    int64_t pitch = pitch_words_for(chunk);
    uint32_t** streams = (uint32_t**)calloc((size_t)(nc ? nc : 1), sizeof(uint32_t*));
    int32_t* nwords = (int32_t*)calloc((size_t)(nc ? nc : 1), sizeof(int32_t));
    uint8_t* first = (uint8_t*)calloc((size_t)(nc ? nc : 1), 1);
    int err = 0;
    int nt = pick_threads(o->n_threads);
    float temp = o->temperature > 0 ? o->temperature : 1.0f;
    /* warm-start: B lanes of S consecutive chunks each (boa.cpp:310-319) */
    int B = 0, S = 1;
    if (o->warm_start && nc > 0) {
        B = o->gpu_batch > 0 ? o->gpu_batch : 64;
        if (B > nc) B = nc;
        S = (nc + B - 1) / B;
    }
    int units = o->warm_start ? B : nc;
#pragma omp parallel for schedule(dynamic, 1) num_threads(nt)
    for (int u = 0; u < units; ++u) {
        ref_state* s = ref_state_new(m, 1);
        for (int i = 0; i < (o->warm_start ? S : 1); ++i) {
            int c = o->warm_start ? u * S + i : u;
            if (c >= nc) break;
            int64_t start = (int64_t)c * chunk;
            int64_t len = n - start < chunk ? n - start : chunk;
            first[c] = len > 0 ? data[start] : 0;
            streams[c] = (uint32_t*)malloc(sizeof(uint32_t) * (size_t)pitch);
            if (!o->warm_start) ref_state_reset(s);
            nwords[c] = len > 1 || o->warm_start
                ? encode_with_state(m, s, data + start, (int32_t)len, o->tile, temp, streams[c],
                                    (int32_t)pitch, o->warm_start)
                : 0;
            if (nwords[c] < 0) err = 1;
        }
        ref_state_free(s);
    }
    if (err) {
        for (int c = 0; c < nc; ++c) free(streams[c]);
        free(streams); free(nwords); free(first);
        return -1;
    }
    int64_t payload = 0;
    for (int c = 0; c < nc; ++c) payload += (int64_t)nwords[c] * 4;
    int64_t cap = 37 + payload + 4 + nc + (int64_t)nc * 10 + 4;
    uint8_t* buf = (uint8_t*)malloc((size_t)cap);
    int64_t p = 0;
    uint32_t u32;
    memcpy(buf + p, "BOA2", 4); p += 4;
    u32 = 1; memcpy(buf + p, &u32, 4); p += 4;
    u32 = o->warm_start ? 1u : 0u; memcpy(buf + p, &u32, 4); p += 4; /* flags */
    uint64_t ps = (uint64_t)processed; memcpy(buf + p, &ps, 8); p += 8;
    u32 = (uint32_t)chunk; memcpy(buf + p, &u32, 4); p += 4;
    u32 = (uint32_t)nc; memcpy(buf + p, &u32, 4); p += 4;
    u32 = (uint32_t)last_len; memcpy(buf + p, &u32, 4); p += 4;
    if (o->warm_start) { /* fp_len 4: the interleave batch (boa.cpp:546-559) */
        buf[p++] = 4;
        u32 = (uint32_t)B; memcpy(buf + p, &u32, 4); p += 4;
    } else {
        buf[p++] = 0;
    }
    for (int c = 0; c < nc; ++c) {
        memcpy(buf + p, streams[c], (size_t)nwords[c] * 4);
        p += (int64_t)nwords[c] * 4;
    }
    int64_t idx = p;
    memcpy(buf + p, "IDX2", 4); p += 4;
    memcpy(buf + p, first, (size_t)nc); p += nc;
    for (int c = 0; c < nc; ++c) p += ref_uvarint_encode((uint64_t)nwords[c] * 4, buf + p);
    u32 = ref_crc32(buf + idx, p - idx);
    memcpy(buf + p, &u32, 4); p += 4;
    for (int c = 0; c < nc; ++c) free(streams[c]);
    free(streams); free(nwords); free(first);
    *out = buf;
    *out_len = p;
    return 0;
}

int32_t ref_decompress(const ref_model* m, const uint8_t* boa, int64_t n, const ref_codec_opts* o,
                       uint8_t** out, int64_t* out_len) {
    ref_boa2_info info;
    int rc = ref_boa2_parse(boa, n, &info, NULL, NULL, NULL);
    if (rc) return rc;
    const int warm = (info.flags & 1u) != 0;
    uint32_t nc = info.n_chunks;
    /* warm-start: the interleave batch comes from the header (boa.cpp:608-610) */
    if (warm && nc > 0 && info.interleave_batch == 0) return -20;
    uint8_t* first = (uint8_t*)malloc(nc ? nc : 1);
    uint64_t* offs = (uint64_t*)malloc(sizeof(uint64_t) * (nc ? nc : 1));
    uint64_t* lens = (uint64_t*)malloc(sizeof(uint64_t) * (nc ? nc : 1));
    rc = ref_boa2_parse(boa, n, &info, first, offs, lens);
    if (rc) { free(first); free(offs); free(lens); return rc; }
    int64_t chunk = info.chunk_len;
    int64_t pitch_bytes = pitch_words_for(chunk) * 4;
    for (uint32_t c = 0; c < nc; ++c)
        if ((int64_t)lens[c] > pitch_bytes) { free(first); free(offs); free(lens); return -9; }
    int64_t total = 0;
    for (uint32_t c = 0; c < nc; ++c)
        total += (c == nc - 1) ? (int64_t)info.last_chunk_len : chunk;
    uint8_t* dst = (uint8_t*)malloc((size_t)(total ? total : 1));
    const uint8_t* payload = boa + info.payload_off;
    enum { GMAX = 8 };
    int nt = pick_threads(o->n_threads);
    /* Units stepped as one group: chunks (cold) or lanes of S chunks (warm).
     * Up to 8 per group, fewer when that would leave threads idle. */
    const int B = warm ? (int)(info.interleave_batch < nc ? info.interleave_batch : nc) : (int)nc;
    const int S = warm && B > 0 ? (int)((nc + (uint32_t)B - 1) / (uint32_t)B) : 1;
    int G = B / (nt > 0 ? nt : 1);
    G = G < 1 ? 1 : (G > GMAX ? GMAX : G);
    int groups = (B + G - 1) / G;
    float inv_t = 1.0f / (o->temperature > 0 ? o->temperature : 1.0f);
#pragma omp parallel num_threads(nt)
    {
        scratch_t sc;
        scratch_init(&sc, m, G);
        ref_state* s = ref_state_new(m, G);
        float* logits = (float*)malloc(sizeof(float) * GMAX * 256);
        uint8_t tok[GMAX];
        ref_rc_dec dec[GMAX];
        uint32_t* words[GMAX];
        int32_t nw[GMAX], len[GMAX];
        uint8_t* o_ptr[GMAX];
        double s_cdf[257];
#pragma omp for schedule(dynamic, 1)
        for (int g = 0; g < groups; ++g) {
            int u0 = g * G, gl = B - u0 < G ? B - u0 : G;
            ref_state_reset(s);
            for (int it = 0; it < S; ++it) {
                /* active lanes lead: unit u runs chunk u*S + it while that is < nc */
                int cnt = 0;
                while (cnt < gl && (int64_t)(u0 + cnt) * S + it < (int64_t)nc) ++cnt;
                if (cnt == 0) break;
                int maxlen = 0;
                for (int i = 0; i < cnt; ++i) {
                    int c = warm ? (u0 + i) * S + it : u0 + i;
                    len[i] = (c == (int)nc - 1) ? (int32_t)info.last_chunk_len : (int32_t)chunk;
                    nw[i] = (int32_t)(lens[c] / 4);
                    words[i] = (uint32_t*)malloc(sizeof(uint32_t) * (size_t)(nw[i] ? nw[i] : 1));
                    memcpy(words[i], payload + offs[c], (size_t)nw[i] * 4);
                    ref_rc_dec_init(&dec[i], words[i], nw[i]);
                    o_ptr[i] = dst + (int64_t)c * chunk;
                    if (len[i] > 0) o_ptr[i][0] = first[c];
                    tok[i] = first[c];
                    if (len[i] > maxlen) maxlen = len[i];
                }
                for (int t = 1; t < maxlen; ++t) {
                    /* step every lane of the group (the reference steps all
                     * lanes each time; finished lanes only stop decoding) */
                    embed_rows(m, tok, cnt, sc.x);
                    for (int l = 0; l < m->L; ++l) block_rows(m, s, l, &sc, cnt, 0, 0);
                    head_rows(m, &sc, cnt, 0, logits);
                    for (int i = 0; i < cnt; ++i) {
                        if (t >= len[i]) continue;
                        ref_cdf_build(logits + (size_t)i * 256, m->hb2, inv_t, s_cdf);
                        uint32_t q = ref_rc_dec_target(&dec[i]);
                        uint32_t lo, hi;
                        int sym = ref_cdf_search(s_cdf, q, &lo, &hi);
                        ref_rc_dec_advance(&dec[i], lo, hi, words[i], nw[i]);
                        o_ptr[i][t] = (uint8_t)sym;
                        tok[i] = (uint8_t)sym;
                    }
                }
                for (int i = 0; i < cnt; ++i) free(words[i]);
                if (warm && it + 1 < S) {
                    /* the lanes that go on consume their chunk's last byte */
                    int next = 0;
                    while (next < cnt && (int64_t)(u0 + next) * S + it + 1 < (int64_t)nc) ++next;
                    if (next > 0) {
                        embed_rows(m, tok, next, sc.x);
                        for (int l = 0; l < m->L; ++l) block_rows(m, s, l, &sc, next, 0, 0);
                    }
                }
            }
        }
        free(logits);
        ref_state_free(s);
        scratch_free(&sc);
    }
    free(first); free(offs); free(lens);
    *out = dst;
    *out_len = total;
    return 0;
}
