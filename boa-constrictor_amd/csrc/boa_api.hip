// Host side of the MI355X codec path: context, weight loader, the compress /
// decompress drivers and the C ABI declared in include/boa_hip.h.
//
// Mirrors portability_solved_cpp/boa.cpp (compress_v2 :280-582, decompress_v2
// :584-817) and boa_gpu.hpp (BoaPredictorGPU :944-1174) for the mambav1
// backbone, on one HIP stream per context.  Differences by design:
//   - bytes stay uint8 end to end (no int32 widening on the host);
//   - the forward of a tile runs on all lanes of a batch at once
//     (M = lanes x tile rows), the coder and the stream compaction run on
//     the device, and only the compacted payload crosses PCIe;
//   - errors are returned as codes, never exit().
#include <hip/hip_runtime.h>

#include <algorithm>
#include <chrono>
#include <cstdio>
#include <cstdlib>
#include <cstring>
#include <mutex>
#include <string>
#include <vector>

#include "../../include/boa_hip.h"
#include "boa_kernels.h"
#include "container.h"

using namespace boa;

namespace boa {
thread_local LaunchTiming g_launch_timing;
}

namespace {

constexpr int VOCAB = 256;

int64_t round_up(int64_t x, int64_t m) { return (x + m - 1) / m * m; }

double now_s() {
  return std::chrono::duration<double>(std::chrono::steady_clock::now().time_since_epoch()).count();
}

struct ProfRec {
  int cls;
  hipEvent_t a, b;
  double work;
};

// Scratch of the allocation-free entry point (boa_forward_chunk_noalloc):
// one fixed array per GPU, held until the process ends.  Host code never
// uses the array's name as an address: boa_create looks up each device's
// own address once (hipGetSymbolAddress, with that device current) and the
// entry point passes that pointer on.  Calls on one GPU share the array.
constexpr size_t kScratchBytes = (size_t)64 << 20;
constexpr int kScratchDevices = 64;
__device__ __align__(256) unsigned char scratch[kScratchBytes];
std::mutex g_scratch_mu;
void* g_scratch_ptr[kScratchDevices] = {};

}  // namespace

struct boa_ctx {
  boa_config cfg{};
  Dims D{};
  hipStream_t own_stream = nullptr;
  hipStream_t stream = nullptr;
  std::string err;
  bool loaded = false;
  float inv_temp = 1.0f;
  int32_t warm_batch = 0;  // warm-start interleave batch; 0 = every chunk starts cold

  // weights (one device allocation)
  bool bf16 = false;  // precision 1: bf16 weights and activations
  float* wbuf = nullptr;
  const float* emb = nullptr;
  const float *hw1 = nullptr, *hb1 = nullptr, *hw2 = nullptr, *hb2 = nullptr;
  std::vector<LayerW> layers;

  // recurrent state for max_lanes lanes
  float* conv_state = nullptr;  // [L][max_lanes][di][4]   (chunk layout)
  float* ssm_state = nullptr;   // [L][max_lanes][di][ds]  (chunk layout)
  // decode step: k-blocked activations and weights (decode.hip) with lane
  // capacity ld_dec, and the recurrent state in step layout (conv
  // [L][di][ld_dec][4], ssm [L][di/16][ds][ld_dec][16]); state_mode says
  // which layout holds the state: 0 chunk, 1 step, 2 both (all zero)
  struct DecW {
    const float *w_in, *w_x, *w_out, *w1, *w2;
    const float* w_dt;  // dt_proj weights, scan quad layout (decode.hip)
    const float* na;    // -exp(A_log) log2(e), scan quad layout
  };
  int n_xdec = 0;  // decode x_proj width: dec_rb(r) + 2 ds
  float* dwbuf = nullptr;
  std::vector<DecW> dlayers;
  // bf16 precision: Linear weights in bf16 for the compress GEMM ([N_pad][K])
  // and the decode GEMM (32-blocked), one allocation
  struct B16W {
    const uint16_t *w_in, *w_x, *w_out, *w1, *w2;
  };
  uint16_t* b16buf = nullptr;
  std::vector<B16W> b16c, b16d;
  const uint16_t *b16c_h1 = nullptr, *b16c_h2 = nullptr, *b16d_h1 = nullptr, *b16d_h2 = nullptr;
  const float *dhw1 = nullptr, *dhw2 = nullptr;
  int ld_dec = 0;
  float* dec_conv = nullptr;
  float* dec_ssm = nullptr;
  int state_mode = 2;
  float *dxt = nullptr, *dxnt = nullptr, *dot = nullptr, *dzt = nullptr, *dcvt = nullptr,
        *ddeltat = nullptr, *dyt = nullptr, *dhidt = nullptr, *dlogits = nullptr;

  // activations
  int64_t rows_cap = 0;
  float *x = nullptr, *xn = nullptr, *xz = nullptr, *cv = nullptr, *delta = nullptr, *y = nullptr,
        *hid = nullptr;
  uint2* lowprob = nullptr;
  // compress: tile k's (low, prob) pairs are coded on enc_stream while tile
  // k + 1's forward pass runs on the caller's stream; the two buffers
  // alternate (lowprob is the one the next forward pass writes)
  uint2* lowprob_alt = nullptr;
  hipStream_t enc_stream = nullptr;
  hipEvent_t lp_ready[2] = {nullptr, nullptr}, lp_free[2] = {nullptr, nullptr};
  hipEvent_t enc_done = nullptr;

  // coder scratch
  int64_t words_cap = 0;  // per-lane pitch x lanes
  uint32_t* words = nullptr;
  RcEnc* enc = nullptr;
  RcDec* dec = nullptr;
  int32_t* sizes = nullptr;
  uint64_t* offsets = nullptr;
  int32_t* lens = nullptr;
  uint8_t* tok = nullptr;
  int* t_counter = nullptr;     // decode step counter (device)

  int n_cus = 0;  // compute units of the device (persistent decode grid)

  // decompress: every step is replayed from a HIP graph on dec_stream; the
  // executable graph is kept while the step's launch arguments stay the same
  hipStream_t dec_stream = nullptr;
  hipEvent_t dec_fork = nullptr, dec_join = nullptr;
  hipGraphExec_t dec_exec = nullptr;
  struct GraphKey {
    int lanes = -1;
    const uint8_t* out = nullptr;
    int64_t stride = 0;
    const uint32_t* payload = nullptr;
    float inv_temp = 0.0f;
    hipStream_t stream = nullptr;
  } dec_key;
  int32_t* h_sizes = nullptr;  // pinned

  // first bytes of the chunks (compress) or of a batch's lanes (decompress)
  uint8_t* first_buf = nullptr;
  int64_t first_cap = 0;
  // warm-start reorder scratch: the staged payload, stream offsets and sizes
  uint32_t* reorder_words = nullptr;
  int64_t reorder_words_cap = 0;
  uint64_t* reorder_off = nullptr;
  int32_t* reorder_sz = nullptr;
  int64_t reorder_n_cap = 0;

  // progress reports (boa.cpp's print_progress)
  boa_progress_fn progress = nullptr;
  void* progress_user = nullptr;
  hipEvent_t prog_ev[2] = {nullptr, nullptr};
  int64_t prog_base = 0, prog_total = 0;  // bytes done before this batch, bytes of the call

  // this device's scratch array (boa_forward_chunk_noalloc), or null
  unsigned char* scratch = nullptr;

  // wall-clock phases of the last buffer call: H2D, device work, D2H (s)
  double t_h2d = 0, t_compute = 0, t_d2h = 0;

  // decode state kept in the caches (bytes; < 0 = the default budget)
  int64_t state_cache_budget = -1;

  // profiling
  bool prof_on = false;
  std::vector<hipEvent_t> ev_pool;
  std::vector<ProfRec> recs;
  double prof_ms[BOA_K_COUNT] = {};
  double prof_work[BOA_K_COUNT] = {};
  int64_t prof_n[BOA_K_COUNT] = {};
};

namespace {

int fail(boa_ctx* c, int code, const std::string& msg) {
  if (c) c->err = msg;
  return code;
}

int hip_fail(boa_ctx* c, hipError_t e, const char* where) {
  return fail(c, BOA_E_HIP, std::string(where) + ": " + hipGetErrorString(e));
}

#define HIP_TRY(c, expr)                                    \
  do {                                                      \
    hipError_t e_ = (expr);                                 \
    if (e_ != hipSuccess) return hip_fail((c), e_, #expr); \
  } while (0)

template <class T>
hipError_t dalloc(T** p, size_t count) {
  *p = nullptr;
  if (!count) count = 1;
  return hipMalloc((void**)p, count * sizeof(T));
}

void dfree(void* p) {
  if (p) (void)hipFree(p);
}

// ---- profiling -------------------------------------------------------------
hipEvent_t take_event(boa_ctx* c) {
  if (c->ev_pool.empty()) {
    hipEvent_t e;
    if (hipEventCreate(&e) != hipSuccess) return nullptr;
    return e;
  }
  hipEvent_t e = c->ev_pool.back();
  c->ev_pool.pop_back();
  return e;
}

void prof_flush(boa_ctx* c) {
  if (c->recs.empty()) return;
  (void)hipEventSynchronize(c->recs.back().b);
  for (auto& r : c->recs) {
    float ms = 0.f;
    if (hipEventElapsedTime(&ms, r.a, r.b) == hipSuccess) c->prof_ms[r.cls] += ms;
    c->prof_n[r.cls] += 1;
    c->prof_work[r.cls] += r.work;
    c->ev_pool.push_back(r.a);
    c->ev_pool.push_back(r.b);
  }
  c->recs.clear();
}

// With profiling on, the launches of f() carry a start / stop event pair in
// their dispatch packets (BOA_LAUNCH): the recorded span is the kernels'
// own, as rocprofv3 measures it, without marker packets between launches.
template <class F>
hipError_t timed(boa_ctx* c, int cls, double work, F&& f) {
  if (!c->prof_on) return f();
  hipEvent_t a = take_event(c), b = take_event(c);
  if (!a || !b) return hipErrorOutOfMemory;
  g_launch_timing = LaunchTiming{a, b, 0};
  hipError_t e = f();
  const int launched = g_launch_timing.launches;
  g_launch_timing = LaunchTiming{};
  if (e != hipSuccess) return e;
  if (launched == 0) {  // nothing was launched (an empty call)
    c->ev_pool.push_back(a);
    c->ev_pool.push_back(b);
    return hipSuccess;
  }
  c->recs.push_back({cls, a, b, work});
  if (c->recs.size() >= 4096) prof_flush(c);
  return hipSuccess;
}

// ---- model dims --------------------------------------------------------------
// The widths the kernels are built for; a model of another d_model (at most
// 512) runs at the next one up, its extra features zero (see Dims).  bf16
// needs widths that are multiples of 64.
int kernel_width(int d, bool bf16) {
  for (int w : {64, 80, 128, 256, 512})
    if (d <= w && !(bf16 && w % 64)) return w;
  return 0;
}

Dims make_dims(const boa_config& cfg) {
  Dims D{};
  D.dn = cfg.d_model;
  D.d = kernel_width(cfg.d_model, cfg.precision == 1);
  D.L = cfg.n_layers;
  D.di = 2 * D.d;
  D.r = (cfg.d_model + 15) / 16;
  D.ds = cfg.d_state;
  D.R = D.r + 2 * D.ds;
  D.ld_in = (int)round_up(2 * D.di, 256);
  D.ld_x = (int)round_up(D.R, 256);
  D.ld_out = (int)round_up(D.d, 256);
  D.ld_1 = (int)round_up(4 * D.d, 256);
  D.ld_2 = (int)round_up(D.d, 256);
  D.ld_h1 = (int)round_up(D.d, 256);
  D.ld_h2 = (int)round_up(VOCAB, 256);
  return D;
}

// compress activation bytes per row: x, xn, xz, conv, delta, y, hidden
// (floats) and the two (low, prob) buffers
int64_t row_bytes(const Dims& D) {
  return 4 * (int64_t)(D.d + D.d + 2 * D.di + D.di + D.R + D.di + 4 * D.d) + 16;
}

int64_t pitch_words_for(int64_t chunk) { return (chunk * 10 + 4096 + 3) / 4; }

int ensure_rows(boa_ctx* c, int64_t rows) {
  if (rows <= c->rows_cap) return BOA_OK;
  const Dims& D = c->D;
  dfree(c->x); dfree(c->xn); dfree(c->xz); dfree(c->cv); dfree(c->delta); dfree(c->y);
  dfree(c->hid); dfree(c->lowprob); dfree(c->lowprob_alt);
  c->rows_cap = 0;
  size_t r = (size_t)rows;
  if (dalloc(&c->x, r * D.d) || dalloc(&c->xn, r * D.d) || dalloc(&c->xz, r * 2 * D.di) ||
      dalloc(&c->cv, r * D.di) || dalloc(&c->delta, r * D.R) || dalloc(&c->y, r * D.di) ||
      dalloc(&c->hid, r * 4 * D.d) || dalloc(&c->lowprob, r) ||
      dalloc(&c->lowprob_alt, r))
    return fail(c, BOA_E_NOMEM, "device allocation of activation buffers failed");
  c->rows_cap = rows;
  return BOA_OK;
}

// The coder stream and its events (created once per context, default priority).
int ensure_enc_stream(boa_ctx* c) {
  hipError_t e = hipSuccess;
  if (!c->enc_stream) e = hipStreamCreateWithFlags(&c->enc_stream, hipStreamNonBlocking);
  for (hipEvent_t* p : {&c->lp_ready[0], &c->lp_ready[1], &c->lp_free[0], &c->lp_free[1],
                        &c->enc_done})
    if (!e && !*p) e = hipEventCreateWithFlags(p, hipEventDisableTiming);
  if (e) return hip_fail(c, e, "coder stream");
  return BOA_OK;
}

int ensure_words(boa_ctx* c, int64_t pitch) {
  const int64_t need = pitch * c->cfg.max_lanes;
  if (need <= c->words_cap) return BOA_OK;
  dfree(c->words);
  c->words_cap = 0;
  if (dalloc(&c->words, (size_t)need)) return fail(c, BOA_E_NOMEM, "device allocation of coder output failed");
  c->words_cap = need;
  return BOA_OK;
}

LayerW layer_at(const boa_ctx* c, int l) { return c->layers[l]; }
float* conv_state_of(boa_ctx* c, int l) {
  return c->conv_state + (size_t)l * c->cfg.max_lanes * c->D.di * 4;
}
float* ssm_state_of(boa_ctx* c, int l) {
  return c->ssm_state + (size_t)l * c->cfg.max_lanes * c->D.di * c->D.ds;
}

#ifndef BOA_LN_FUSE
#define BOA_LN_FUSE 1
#endif

hipError_t gemm(boa_ctx* c, const float* X, int ldx, const float* W, int ldw, float* C, int ldc,
                const float* bias, const float* res, int ldr, int M, int N, int K, int act) {
  GemmArgs a{X, ldx, W, ldw, C, ldc, bias, res, ldr, M, N, K, act};
  const int cls = gemm_f32_config(a) == 0 ? BOA_K_GEMM : BOA_K_GEMM_SMALL;
  return timed(c, cls, 2.0 * M * N * K, [&] { return gemm_f32(a, c->stream); });
}

// A 256-wide fp32 GEMM with the next LayerNorm in its epilogue (mode 1: LN1
// of acc + bias + res, which also goes to C; mode 2: LN2 of acc + bias).
hipError_t gemm_ln(boa_ctx* c, const float* X, int ldx, const float* W, int ldw, float* C, int ldc,
                   const float* bias, const float* res, int ldr, int M, int K, const float* ln_w,
                   const float* ln_b, float* out, int mode) {
  GemmArgs a{X, ldx, W, ldw, C, ldc, bias, res, ldr, M, 256, K, ACT_NONE};
  const LnEpi ln{ln_w, ln_b, out, 256, mode, c->D.dn};
  return timed(c, BOA_K_GEMM, 2.0 * M * 256 * K, [&] { return gemm_f32_ln(a, ln, c->stream); });
}

// bf16 GEMM of the compress pass: X bf16 [M][K], W bf16 [N_pad][K].
hipError_t gemmb(boa_ctx* c, const void* X, const uint16_t* W, void* C, int ldc, bool c_bf16,
                 uint16_t* C2, const float* bias, const float* res, int ldr, int M, int N, int K,
                 int act) {
  GemmB16Args a{(const uint16_t*)X, K, W, K, C, ldc, c_bf16 ? 1 : 0, C2, bias, res, ldr, M, N, K,
                act};
  const int cls = N >= 256 ? BOA_K_GEMM : BOA_K_GEMM_SMALL;
  return timed(c, cls, 2.0 * M * N * K, [&] { return gemm_bf16(a, c->stream); });
}

// bf16 block (precision 1): the fp32 block's sequence with bf16 activations
// (xn, xz, conv, delta, y, out_proj output, hid) and fp32 x; the last layer's
// FF2 also stores a bf16 copy of x (into y's buffer) for head1.
hipError_t block_forward_b16(boa_ctx* c, int l, int rows, int lanes, int T, const TokenSrc& tok0,
                             int t0) {
  const Dims& D = c->D;
  const LayerW W = layer_at(c, l);
  const boa_ctx::B16W& B = c->b16c[l];
  hipStream_t s = c->stream;
  const double ln_bytes = 3.0 * 4 * rows * D.d;
  // d_model 256 (the fused FF kernel, whole rows per block): LN2 runs in its
  // prologue and the next layer's LN1 in its epilogue
  const bool fuse_ln = BOA_LN_FUSE && D.d == 256;
  hipError_t e = hipSuccess;
  if (l == 0 || !fuse_ln)
    e = timed(c, BOA_K_LN, ln_bytes, [&] {
      return l == 0 ? launch_ln1(c->emb, tok0, T, t0, c->x, c->xn, W.ln1_w, W.ln1_b, rows, D.d,
                                 D.dn, true, s)
                    : launch_ln1(nullptr, TokenSrc{nullptr, 0, 0, 0}, T, t0, c->x, c->xn,
                                 W.ln1_w, W.ln1_b, rows, D.d, D.dn, true, s);
    });
  if (!e) e = gemmb(c, c->xn, B.w_in, c->xz, 2 * D.di, true, nullptr, W.b_in, nullptr, 0, rows,
                    2 * D.di, D.d, ACT_NONE);
  if (!e)
    e = timed(c, BOA_K_CONV, 2.0 * rows * D.di * 2, [&] {
      return launch_conv_chunk(c->xz, conv_state_of(c, l), W.conv_w, W.conv_b, c->cv, lanes, T,
                               D.di, true, s);
    });
  if (!e) e = gemmb(c, c->cv, B.w_x, c->delta, D.R, true, nullptr, nullptr, nullptr, 0, rows, D.R,
                    D.di, ACT_NONE);
  if (!e)
    e = timed(c, BOA_K_SCAN, 2.0 * rows * (3.0 * D.di + D.R), [&] {
      return launch_scan_chunk(D, W, c->xz, c->cv, c->delta, ssm_state_of(c, l), c->y, lanes, T,
                               true, s);
    });
  if (!e) e = gemmb(c, c->y, B.w_out, c->xn, D.d, true, nullptr, W.b_out, nullptr, 0, rows, D.d,
                    D.di, ACT_NONE);
  if (!e && !fuse_ln)
    e = timed(c, BOA_K_LN, 2.0 * 2 * rows * D.d,
              [&] { return launch_ln2(c->xn, c->xn, W.ln2_w, W.ln2_b, rows, D.d, D.dn, true, s); });
  // d_model 256: FF1 + GELU + FF2 in one kernel, the hidden layer kept in
  // LDS (MI355X, C3 probe: bf16 GEMMs 131.9 -> 125.1 ms, compress 17.52 ->
  // 18.07 MB/s).  At d_model 512 the fused form, with 64-row blocks that
  // re-read both weight matrices per block, was slower (553 -> 707 ms).
  if (D.d == 256) {
    if (e) return e;
    FfnB16Args f{(const uint16_t*)c->xn, B.w1, B.w2, W.b1, W.b2, c->x, c->x,
                 l == D.L - 1 ? (uint16_t*)c->y : nullptr, rows, D.d};
    f.n = D.dn;
    if (fuse_ln) {
      f.ln2_w = W.ln2_w;
      f.ln2_b = W.ln2_b;
      if (l + 1 < D.L) {
        const LayerW Wn = layer_at(c, l + 1);
        f.ln1_w = Wn.ln1_w;
        f.ln1_b = Wn.ln1_b;
        f.xn = (uint16_t*)c->xn;
      }
    }
    return timed(c, BOA_K_GEMM, 2.0 * rows * 8.0 * D.d * D.d, [&] { return ffn_bf16(f, s); });
  }
  if (!e) e = gemmb(c, c->xn, B.w1, c->hid, 4 * D.d, true, nullptr, W.b1, nullptr, 0, rows, 4 * D.d,
                    D.d, ACT_GELU);
  if (!e)
    e = gemmb(c, c->hid, B.w2, c->x, D.d, false, l == D.L - 1 ? (uint16_t*)c->y : nullptr, W.b2,
              c->x, D.d, rows, D.d, 4 * D.d, ACT_NONE);
  return e;
}

// One mambav1 block on `rows` = lanes x T rows (boa_gpu.hpp:895-902):
// res = x; x = LN1(x); x = Mamba(x); x = LN2(x); x = FF(x) + res.
// x keeps the residual, LN1 writes xn, out_proj writes xn.
hipError_t block_forward(boa_ctx* c, int l, int rows, int lanes, int T, const TokenSrc& tok0,
                         int t0) {
  const Dims& D = c->D;
  const LayerW W = layer_at(c, l);
  hipStream_t s = c->stream;
  hipError_t e;
  const double ln_bytes = 3.0 * 4 * rows * D.d;
  // d_model 256 in 128 x 256 tiles: LN2 runs in out_proj's epilogue and the
  // next layer's LN1 in FF2's (the rows are whole in one block)
  const bool fuse_ln = BOA_LN_FUSE && D.d == 256 && gemm_f32_config(GemmArgs{
      nullptr, 0, nullptr, 0, nullptr, 0, nullptr, nullptr, 0, rows, 256, 256, ACT_NONE}) == 0;
  if (l == 0 || !fuse_ln) {
    e = timed(c, BOA_K_LN, ln_bytes, [&] {
      return l == 0 ? launch_ln1(c->emb, tok0, T, t0, c->x, c->xn, W.ln1_w, W.ln1_b, rows, D.d,
                                 D.dn, false, s)
                    : launch_ln1(nullptr, TokenSrc{nullptr, 0, 0, 0}, T, t0, c->x, c->xn,
                                 W.ln1_w, W.ln1_b, rows, D.d, D.dn, false, s);
    });
    if (e) return e;
  }
  if ((e = gemm(c, c->xn, D.d, W.w_in, D.ld_in, c->xz, 2 * D.di, W.b_in, nullptr, 0, rows,
                2 * D.di, D.d, ACT_NONE)))
    return e;
  const double conv_bytes = 4.0 * rows * D.di * 2;
  e = timed(c, BOA_K_CONV, conv_bytes, [&] {
    return launch_conv_chunk(c->xz, conv_state_of(c, l), W.conv_w, W.conv_b, c->cv, lanes, T,
                             D.di, false, s);
  });
  if (e) return e;
  if ((e = gemm(c, c->cv, D.di, W.w_x, D.ld_x, c->delta, D.R, nullptr, nullptr, 0, rows, D.R, D.di,
                ACT_NONE)))
    return e;
  // algorithmic bytes: u, z, y per element, the delta row per token
  const double scan_bytes = 4.0 * rows * (3.0 * D.di + D.R);
  e = timed(c, BOA_K_SCAN, scan_bytes, [&] {
    return launch_scan_chunk(D, W, c->xz, c->cv, c->delta, ssm_state_of(c, l), c->y, lanes, T,
                             false, s);
  });
  if (e) return e;
  if (fuse_ln) {
    if ((e = gemm_ln(c, c->y, D.di, W.w_out, D.ld_out, nullptr, 0, W.b_out, nullptr, 0, rows, D.di,
                     W.ln2_w, W.ln2_b, c->xn, 2)))
      return e;
  } else {
    if ((e = gemm(c, c->y, D.di, W.w_out, D.ld_out, c->xn, D.d, W.b_out, nullptr, 0, rows, D.d,
                  D.di, ACT_NONE)))
      return e;
    e = timed(c, BOA_K_LN, ln_bytes,
              [&] { return launch_ln2(c->xn, c->xn, W.ln2_w, W.ln2_b, rows, D.d, D.dn, false, s); });
    if (e) return e;
  }
  if ((e = gemm(c, c->xn, D.d, W.w1, D.ld_1, c->hid, 4 * D.d, W.b1, nullptr, 0, rows, 4 * D.d, D.d,
                ACT_GELU)))
    return e;
  if (fuse_ln && l + 1 < D.L) {
    const LayerW Wn = layer_at(c, l + 1);
    return gemm_ln(c, c->hid, 4 * D.d, W.w2, D.ld_2, c->x, D.d, W.b2, c->x, D.d, rows, 4 * D.d,
                   Wn.ln1_w, Wn.ln1_b, c->xn, 1);
  }
  return gemm(c, c->hid, 4 * D.d, W.w2, D.ld_2, c->x, D.d, W.b2, c->x, D.d, rows, D.d, 4 * D.d,
              ACT_NONE);
}

hipError_t head_forward(boa_ctx* c, int rows, bool add_bias, float* logits) {
  const Dims& D = c->D;
  if (c->bf16) {  // head1 reads the bf16 copy of x stored in y's buffer
    hipError_t e = gemmb(c, c->y, c->b16c_h1, c->xn, D.d, true, nullptr, c->hb1, nullptr, 0, rows,
                         D.d, D.d, ACT_RELU);
    if (e) return e;
    return gemmb(c, c->xn, c->b16c_h2, logits, VOCAB, false, nullptr, add_bias ? c->hb2 : nullptr,
                 nullptr, 0, rows, VOCAB, D.d, ACT_NONE);
  }
  hipError_t e = gemm(c, c->x, D.d, c->hw1, D.ld_h1, c->xn, D.d, c->hb1, nullptr, 0, rows, D.d, D.d,
                      ACT_RELU);
  if (e) return e;
  return gemm(c, c->xn, D.d, c->hw2, D.ld_h2, logits, VOCAB, add_bias ? c->hb2 : nullptr, nullptr, 0,
              rows, VOCAB, D.d, ACT_NONE);
}

hipError_t ensure_state_layout(boa_ctx* c, int want_step);

hipError_t blocks_forward(boa_ctx* c, const TokenSrc& tok, int lanes, int T, int t0) {
  const int rows = lanes * T;
  hipError_t es = ensure_state_layout(c, 0);
  if (es) return es;
  for (int l = 0; l < c->D.L; ++l) {
    hipError_t e = c->bf16 ? block_forward_b16(c, l, rows, lanes, T, tok, t0)
                           : block_forward(c, l, rows, lanes, T, tok, t0);
    if (e) return e;
  }
  return hipSuccess;
}

hipError_t forward_tile(boa_ctx* c, const TokenSrc& tok, int lanes, int T, int t0, float* logits) {
  hipError_t e = blocks_forward(c, tok, lanes, T, t0);
  return e ? e : head_forward(c, lanes * T, true, logits);
}

// A compress tile up to the coder's input: the blocks, head.1, then head.2
// fused with the CDF, which writes each row's (low, prob) of the next byte to
// c->lowprob without storing the logits.
hipError_t forward_tile_cdf(boa_ctx* c, const TokenSrc& tok, int lanes, int T, int t0) {
  const Dims& D = c->D;
  const int rows = lanes * T;
  hipError_t e = blocks_forward(c, tok, lanes, T, t0);
  if (c->bf16) {  // head1 reads the bf16 copy of x stored in y's buffer
    if (!e)
      e = gemmb(c, c->y, c->b16c_h1, c->xn, D.d, true, nullptr, c->hb1, nullptr, 0, rows, D.d,
                D.d, ACT_RELU);
    if (e) return e;
    GemmB16Args a{(const uint16_t*)c->xn, D.d, c->b16c_h2, D.d, nullptr, 0, 0, nullptr, c->hb2,
                  nullptr, 0, rows, VOCAB, D.d, ACT_NONE};
    CdfEpi ce{tok.base, tok.stride, tok.total, tok.len, T, t0, c->inv_temp, c->lowprob};
    return timed(c, BOA_K_HEAD_CDF, 2.0 * rows * VOCAB * D.d,
                 [&] { return gemm_bf16_head_cdf(a, ce, c->stream); });
  }
  if (!e)
    e = gemm(c, c->x, D.d, c->hw1, D.ld_h1, c->xn, D.d, c->hb1, nullptr, 0, rows, D.d, D.d,
             ACT_RELU);
  if (e) return e;
  GemmArgs a{c->xn, D.d, c->hw2, D.ld_h2, nullptr, 0, c->hb2, nullptr, 0, rows, VOCAB, D.d,
             ACT_NONE};
  CdfEpi ce{tok.base, tok.stride, tok.total, tok.len, T, t0, c->inv_temp, c->lowprob};
  return timed(c, BOA_K_HEAD_CDF, 2.0 * rows * VOCAB * D.d,
               [&] { return gemm_f32_head_cdf(a, ce, c->stream); });
}

float* dec_conv_of(boa_ctx* c, int l) {
  return c->dec_conv + (size_t)l * c->D.di * c->ld_dec * 4;
}
float* dec_ssm_of(boa_ctx* c, int l) {
  return c->dec_ssm + (size_t)l * c->D.di * c->D.ds * c->ld_dec;
}

// W is a k-blocked decode weight with lane capacity round_up(N, 16).
hipError_t dgemm(boa_ctx* c, const float* Xt, const float* W, float* C, int ldc,
                 const float* bias, const float* res, int M, int N, int K, int act,
                 int row_major = 0) {
  DecGemmArgs a{};
  a.Xt = Xt; a.ldx = c->ld_dec; a.W = W; a.ldw = (int)round_up(N, 16); a.C = C; a.ldc = ldc;
  a.bias = bias;
  a.res = res; a.ldr = c->ld_dec; a.M = M; a.N = N; a.K = K; a.act = act; a.row_major = row_major;
  return timed(c, BOA_K_DEC_GEMM, 2.0 * M * N * K, [&] { return dec_gemm(a, c->stream); });
}

// Move the recurrent state into the layout the next call needs.
hipError_t ensure_state_layout(boa_ctx* c, int want_step) {
  if (c->state_mode == 2 || c->state_mode == want_step) {
    c->state_mode = want_step;
    return hipSuccess;
  }
  const Dims& D = c->D;
  for (int l = 0; l < D.L; ++l) {
    hipError_t e = want_step
        ? launch_state_relayout(conv_state_of(c, l), ssm_state_of(c, l), dec_conv_of(c, l),
                                dec_ssm_of(c, l), c->cfg.max_lanes, D.di, D.ds, c->ld_dec, true,
                                c->bf16, c->stream)
        : launch_state_relayout(dec_conv_of(c, l), dec_ssm_of(c, l), conv_state_of(c, l),
                                ssm_state_of(c, l), c->cfg.max_lanes, D.di, D.ds, c->ld_dec, false,
                                c->bf16, c->stream);
    if (e) return e;
  }
  c->state_mode = want_step;
  return hipSuccess;
}

// One decode step for lanes [lane0, lane0 + lanes) on the k-blocked buffers
// (the mambav1 block of boa_gpu.hpp:834-843 and the head of :1048-1052),
// ordered on stream s; layer 0's LN1 advances *t_counter.  The causal conv
// step runs in in_proj's epilogue.  Logits are written row-major [lane][256]
// (logits points at lane 0 of the range).  The state must be in step layout.
// Layers whose decode state (SSM and conv) goes through the caches: as many
// as fit in 160 MiB, the rest of the 256 MB last-level cache being left to
// the weights and activations; the state of the other layers is streamed
// past the caches.  At C2 (1000 lanes, 40 KB of state per lane and layer)
// this caches 4 of 8 layers: decode 1.72 -> 1.78 MB/s on MI355X, against
// 1.75 with 5 and 1.65 with all 8.
constexpr int64_t kStateCacheBudget = (int64_t)160 << 20;

int dec_cached_layers(const boa_ctx* c, int lanes) {
  const double per_layer = (double)lanes * c->D.di * (c->D.ds + 4) * sizeof(float);
  const double budget =
      (double)(c->state_cache_budget >= 0 ? c->state_cache_budget : kStateCacheBudget);
  return per_layer <= 0 ? c->D.L : std::min(c->D.L, (int)(budget / per_layer));
}

// LayerNorm fused into in_proj and FF1 up to 2048 lanes; above that the
// separate kernels spread the work better (MI355X sweep)
bool dec_fuse_ln(const boa_ctx* c, int lanes) {
  const Dims& D = c->D;
  return lanes <= 2048 && dec_ln_gemm_fits(D.d, 2 * D.di) && dec_ln_gemm_fits(D.d, 4 * D.d);
}

// x_proj fused into the scan kernel up to 2048 lanes (its x_proj is
// recomputed by the 4 channel blocks of a lane tile); above that the
// separate x_proj GEMM is faster (MI355X, C2 probe at 1000 lanes: decode
// 1.806 -> 1.852 MB/s fused; C4 probe at 4096 lanes: 2.673 -> 2.527 fused).
bool dec_fuse_xproj(const boa_ctx* c, int lanes) {
  return lanes <= 2048 && dec_xscan_fits(c->D);
}

// head.2 fused with the coder step from 2048 lanes on: its 16-lane blocks
// (one per 16 lanes) fill the CUs only there (MI355X: C2 probe at 1000 lanes
// 1.865 MB/s apart against 1.852 fused; C4 probe at 4096 lanes 2.514
// apart against 2.527 fused).
bool dec_fuse_head(int lanes) { return lanes >= 2048; }

// Grow-only device buffer: reallocated only when a call needs more.
template <class T>
hipError_t ensure_buf(T** p, int64_t* cap, int64_t need) {
  if (need <= *cap) return hipSuccess;
  dfree(*p);
  *p = nullptr;
  *cap = 0;
  hipError_t e = dalloc(p, (size_t)need);
  if (e == hipSuccess) *cap = need;
  return e;
}

// Drop the cached decode graph (its kernels hold weight and buffer pointers
// and template choices that a weight load or a cache-budget change alters).
void drop_dec_graph(boa_ctx* c) {
  if (!c->dec_exec) return;
  if (c->dec_stream) (void)hipStreamSynchronize(c->dec_stream);
  (void)hipGraphExecDestroy(c->dec_exec);
  c->dec_exec = nullptr;
  c->dec_key = boa_ctx::GraphKey{};
}

// Report progress to the caller's callback once the work before the last
// marker has finished on the device: `done` bytes of `total` are reported
// when the marker recorded at the previous call has completed, so one
// slice of work stays queued while the host waits.
hipError_t progress_mark(boa_ctx* c, int phase, int64_t done_prev, int64_t total, int64_t* pend,
                         int* slot) {
  if (!c->progress) return hipSuccess;
  for (int k = 0; k < 2; ++k)
    if (!c->prog_ev[k]) {
      hipError_t e = hipEventCreateWithFlags(&c->prog_ev[k], hipEventDisableTiming);
      if (e) return e;
    }
  hipError_t e = hipEventRecord(c->prog_ev[*slot], c->stream);
  if (e) return e;
  if (*pend >= 0) {
    e = hipEventSynchronize(c->prog_ev[*slot ^ 1]);
    if (e) return e;
    c->progress(c->progress_user, phase, *pend, total);
  }
  *pend = done_prev;
  *slot ^= 1;
  return hipSuccess;
}

hipError_t step_range_b16(boa_ctx* c, int lane0, int lanes, hipStream_t s, int* t_counter,
                          const uint8_t* tok, bool add_bias, float* logits);

// with_head2 = false stops after head.1 (its output in the k-blocked dot
// buffer): the decode loop runs head.2 fused with the coder step.
hipError_t step_range(boa_ctx* c, int lane0, int lanes, hipStream_t s, int* t_counter,
                      const uint8_t* tok, bool add_bias, float* logits, bool with_head2 = true) {
  if (c->bf16) return step_range_b16(c, lane0, lanes, s, t_counter, tok, add_bias, logits);
  const Dims& D = c->D;
  const int ld = c->ld_dec;
  const size_t a0 = (size_t)lane0 * 16;  // k-blocked activations
  float *xt = c->dxt + a0, *xnt = c->dxnt + a0, *ot = c->dot + a0, *zt = c->dzt + a0,
        *cvt = c->dcvt + a0, *rows = c->ddeltat + a0, *yt = c->dyt + a0, *hidt = c->dhidt + a0;
  hipStream_t saved = c->stream;
  c->stream = s;  // dgemm and timed() launch on c->stream
  hipError_t e = hipSuccess;
  const bool fuse_ln = dec_fuse_ln(c, lanes);
  const int n_cached = dec_cached_layers(c, lanes);
  for (int l = 0; l < D.L && !e; ++l) {
    const LayerW& W = c->layers[l];
    const boa_ctx::DecW& DW = c->dlayers[l];
    float* conv = dec_conv_of(c, l) + (size_t)lane0 * 4;
    float* ssm = dec_ssm_of(c, l) + (size_t)lane0 * 64;
    const bool cached = l < n_cached;
    DecGemmArgs a{};
    a.state_cached = cached ? 1 : 0;
    a.Xt = xnt; a.ldx = ld; a.W = DW.w_in; a.ldw = 2 * D.di; a.C = zt; a.ldc = ld;
    a.bias = W.b_in; a.M = lanes; a.N = 2 * D.di; a.K = D.d; a.act = ACT_NONE;
    a.conv_di = D.di; a.conv_state = conv; a.ld_state = ld; a.conv_w = W.conv_w;
    a.conv_b = W.conv_b; a.conv_out = cvt; a.ln_n = D.dn;
    if (fuse_ln) {  // LN1 in front of in_proj, in one kernel
      a.Xt = xt;
      e = timed(c, BOA_K_DEC_LNGEMM, 2.0 * lanes * a.N * a.K, [&] {
        return launch_dec_ln_gemm(1, a, l == 0 ? c->emb : nullptr, tok, xt, W.ln1_w, W.ln1_b,
                                  l == 0 ? t_counter : nullptr, s);
      });
    } else {
      e = timed(c, BOA_K_LN, 3.0 * 4 * lanes * D.d, [&] {
        return launch_dec_ln1(l == 0 ? c->emb : nullptr, tok, xt, xnt, W.ln1_w, W.ln1_b, lanes,
                              D.d, D.dn, ld, l == 0 ? t_counter : nullptr, s);
      });
      if (!e)
        e = timed(c, BOA_K_DEC_GEMM, 2.0 * lanes * a.N * a.K, [&] { return dec_gemm(a, s); });
    }
    if (!e && dec_fuse_xproj(c, lanes)) {  // x_proj inside the scan kernel
      e = timed(c, BOA_K_DEC_SCAN, 8.0 * lanes * D.di * D.ds + 4.0 * lanes * (3.0 * D.di + D.R), [&] {
        return launch_dec_xscan(D, W, DW.na, DW.w_dt, DW.w_x, (int)round_up(c->n_xdec, 16), zt, cvt,
                                ssm, yt, lanes, ld, ld, cached, s);
      });
    } else if (!e) {
      e = dgemm(c, cvt, DW.w_x, rows, ld, nullptr, nullptr, lanes, c->n_xdec, D.di, ACT_NONE);
      if (!e)
        e = timed(c, BOA_K_DEC_SCAN, 8.0 * lanes * D.di * D.ds + 4.0 * lanes * (3.0 * D.di + D.R), [&] {
          return launch_dec_scan(D, W, DW.na, DW.w_dt, zt, cvt, rows, ssm, yt, lanes, ld, ld, cached, s);
        });
    }
    if (!e) e = dgemm(c, yt, DW.w_out, ot, ld, W.b_out, nullptr, lanes, D.d, D.di, ACT_NONE);
    if (!e && fuse_ln) {  // LN2 in front of FF1, in one kernel
      DecGemmArgs f{};
      f.Xt = ot; f.ldx = ld; f.W = DW.w1; f.ldw = 4 * D.d; f.C = hidt; f.ldc = ld;
      f.bias = W.b1; f.M = lanes; f.N = 4 * D.d; f.K = D.d; f.act = ACT_GELU; f.ln_n = D.dn;
      e = timed(c, BOA_K_DEC_LNGEMM, 2.0 * lanes * f.N * f.K, [&] {
        return launch_dec_ln_gemm(2, f, nullptr, nullptr, nullptr, W.ln2_w, W.ln2_b, nullptr, s);
      });
    } else if (!e) {
      e = timed(c, BOA_K_LN, 3.0 * 4 * lanes * D.d,
                [&] { return launch_dec_ln2(ot, xnt, W.ln2_w, W.ln2_b, lanes, D.d, D.dn, ld, s); });
      if (!e) e = dgemm(c, xnt, DW.w1, hidt, ld, W.b1, nullptr, lanes, 4 * D.d, D.d, ACT_GELU);
    }
    if (!e) e = dgemm(c, hidt, DW.w2, xt, ld, W.b2, xt, lanes, D.d, 4 * D.d, ACT_NONE);
  }
  if (!e) e = dgemm(c, xt, c->dhw1, ot, ld, c->hb1, nullptr, lanes, D.d, D.d, ACT_RELU);
  if (!e && with_head2)
    e = dgemm(c, ot, c->dhw2, logits, VOCAB, add_bias ? c->hb2 : nullptr, nullptr, lanes, VOCAB,
              D.d, ACT_NONE, 1);
  c->stream = saved;
  return e;
}

// bf16 decode step: bf16 32-blocked activations, fp32 k-blocked x; the
// last layer's FF2 also writes x in bf16 (into y's buffer) for head1.
hipError_t step_range_b16(boa_ctx* c, int lane0, int lanes, hipStream_t s, int* t_counter,
                          const uint8_t* tok, bool add_bias, float* logits) {
  const Dims& D = c->D;
  const int ld = c->ld_dec;
  const size_t a0 = (size_t)lane0 * 32;  // bf16 32-blocked activations
  float* xt = c->dxt + (size_t)lane0 * 16;
  uint16_t *xnt = (uint16_t*)c->dxnt + a0, *ot = (uint16_t*)c->dot + a0,
           *zt = (uint16_t*)c->dzt + a0, *cvt = (uint16_t*)c->dcvt + a0,
           *rows = (uint16_t*)c->ddeltat + a0, *yt = (uint16_t*)c->dyt + a0,
           *hidt = (uint16_t*)c->dhidt + a0;
  auto g = [&](const uint16_t* X, const uint16_t* W, int N, int K, void* C, int mode,
               const float* bias, int act) {
    DecB16Args a{};
    a.X = X; a.ldx = ld; a.W = W; a.ldw = (int)round_up(N, 16); a.C = C; a.ldc = ld;
    a.out_mode = mode; a.bias = bias; a.M = lanes; a.N = N; a.K = K; a.act = act;
    a.n_cus = c->n_cus;
    return a;
  };
  auto run = [&](const DecB16Args& a) {
    return timed(c, BOA_K_DEC_GEMM, 2.0 * a.M * a.N * a.K, [&] { return dec_b16_gemm(a, s); });
  };
  hipError_t e = hipSuccess;
  const int n_cached = dec_cached_layers(c, lanes);
  for (int l = 0; l < D.L && !e; ++l) {
    const LayerW& W = c->layers[l];
    const boa_ctx::DecW& DW = c->dlayers[l];
    const boa_ctx::B16W& B = c->b16d[l];
    // the conv state of bf16 is four bf16 (two floats' bytes) per channel and lane
    float* conv = dec_conv_of(c, l) + (size_t)lane0 * 2;
    float* ssm = dec_ssm_of(c, l) + (size_t)lane0 * 64;
    const bool cached = l < n_cached;
    e = timed(c, BOA_K_LN, 3.0 * 4 * lanes * D.d, [&] {
      return launch_dec_b16_ln1(l == 0 ? c->emb : nullptr, tok, xt, xnt, W.ln1_w, W.ln1_b, lanes,
                                D.d, D.dn, ld, l == 0 ? t_counter : nullptr, s);
    });
    if (!e) {
      DecB16Args a = g(xnt, B.w_in, 2 * D.di, D.d, zt, DEC_OUT_B16, W.b_in, ACT_NONE);
      a.conv_di = D.di; a.conv_state = conv; a.ld_state = ld; a.conv_w = W.conv_w;
      a.conv_b = W.conv_b; a.conv_out = cvt; a.state_cached = cached ? 1 : 0;
      e = run(a);
    }
    if (!e) e = run(g(cvt, B.w_x, c->n_xdec, D.di, rows, DEC_OUT_B16, nullptr, ACT_NONE));
    if (!e)
      e = timed(c, BOA_K_DEC_SCAN, 8.0 * lanes * D.di * D.ds + 2.0 * lanes * (3.0 * D.di + D.R), [&] {
        return launch_dec_b16_scan(D, W, DW.na, DW.w_dt, zt, cvt, rows, ssm, yt, lanes, ld, ld, cached,
                                  s);
      });
    if (!e) e = run(g(yt, B.w_out, D.d, D.di, ot, DEC_OUT_B16, W.b_out, ACT_NONE));
    if (!e)
      e = timed(c, BOA_K_LN, 2.0 * 2 * lanes * D.d,
                [&] { return launch_dec_b16_ln2(ot, xnt, W.ln2_w, W.ln2_b, lanes, D.d, D.dn, ld, s); });
    if (!e) e = run(g(xnt, B.w1, 4 * D.d, D.d, hidt, DEC_OUT_B16, W.b1, ACT_GELU));
    if (!e) {
      DecB16Args a = g(hidt, B.w2, D.d, 4 * D.d, xt, DEC_OUT_F32, W.b2, ACT_NONE);
      a.res = xt; a.ldr = ld;
      if (l == D.L - 1) a.C2 = yt;
      e = run(a);
    }
  }
  if (!e) e = run(g(yt, c->b16d_h1, D.d, D.d, ot, DEC_OUT_B16, c->hb1, ACT_RELU));
  if (!e) {
    DecB16Args a = g(ot, c->b16d_h2, VOCAB, D.d, logits, DEC_OUT_ROWMAJOR,
                     add_bias ? c->hb2 : nullptr, ACT_NONE);
    a.ldc = VOCAB;
    e = run(a);
  }
  return e;
}

hipError_t step_forward(boa_ctx* c, const uint8_t* tok, int lanes, bool add_bias, float* logits) {
  hipError_t e = ensure_state_layout(c, 1);
  if (e) return e;
  return step_range(c, 0, lanes, c->stream, c->t_counter, tok, add_bias, logits);
}

int check_ready(boa_ctx* c) {
  if (!c) return BOA_E_ARG;
  if (!c->loaded) return fail(c, BOA_E_STATE, "no weights loaded");
  return BOA_OK;
}

int64_t auto_tile(const boa_ctx* c, int64_t chunk, int lanes) {
  if (c->cfg.tile > 0) return std::min<int64_t>(c->cfg.tile, chunk);
  const int64_t budget = (int64_t)24 << 30;
  int64_t rows = budget / row_bytes(c->D);
  int64_t T = rows / std::max(lanes, 1);
  T = std::max<int64_t>(64, T / 64 * 64);
  T = std::min<int64_t>(T, 2048);
  return std::min<int64_t>(T, chunk);
}

__global__ void gather_first_kernel(const uint8_t* base, int64_t stride, int64_t total, int lanes,
                                    uint8_t* first) {
  int b = blockIdx.x * blockDim.x + threadIdx.x;
  if (b >= lanes) return;
  int64_t pos = (int64_t)b * stride;
  first[b] = pos < total ? base[pos] : 0;
}

__global__ void na2_kernel(const float* a_log, float* out, int n) {
  int i = blockIdx.x * blockDim.x + threadIdx.x;
  if (i < n) out[i] = scan_na2(a_log[i]);
}

__global__ void decode_init_kernel(const uint8_t* first, const int32_t* lens, uint8_t* tok,
                                   uint8_t* out, int64_t out_stride, int lanes, int* t_counter) {
  int b = blockIdx.x * blockDim.x + threadIdx.x;
  if (b == 0) *t_counter = 0;
  if (b >= lanes) return;
  tok[b] = first[b];
  if (lens[b] > 0) out[(size_t)b * out_stride] = first[b];
}

// ---- weight parsing ----------------------------------------------------------
struct HostReader {
  const uint8_t* p;
  size_t n, pos;
  bool fp16, bad;
  void vec(std::vector<float>& dst, size_t count) {
    dst.resize(count);
    const size_t esz = fp16 ? 2 : 4;
    if (bad || pos + count * esz > n) { bad = true; return; }
    if (fp16) {
      for (size_t i = 0; i < count; ++i) {
        uint16_t h;
        memcpy(&h, p + pos + 2 * i, 2);
        dst[i] = boa_host_half_to_float(h);
      }
    } else {
      memcpy(dst.data(), p + pos, count * 4);
    }
    pos += count * esz;
  }
};

}  // namespace

namespace {

// Steps 1 .. maxlen-1 of a batch.  Every step is the same launch sequence
// (the step counter lives on the device), so it is captured once into a HIP
// graph on the decode stream and replayed; the decode stream is ordered
// after, and the context stream after it, by events.  With profiling on, the
// steps are launched directly on the context stream.
hipError_t decode_steps(boa_ctx* c, int lanes, int maxlen, uint8_t* out, int64_t chunk,
                        const uint32_t* d_payload) {
  hipStream_t s = c->stream;
  const Dims& D = c->D;
  if (!c->bf16 && dec_persist_fits(D.d, D.ds, D.r, D.L)) {
    // small model: every step in one persistent kernel (decode_persist.hip)
    PersistArgs p{};
    for (int l = 0; l < D.L; ++l) {
      const LayerW& W = c->layers[l];
      const boa_ctx::DecW& DW = c->dlayers[l];
      p.layer[l] = PersistLayer{W.ln1_w, W.ln1_b, DW.w_in, W.b_in, W.conv_w, W.conv_b, DW.w_x,
                                DW.na, DW.w_dt, W.b_dt, W.dd, DW.w_out, W.b_out, W.ln2_w,
                                W.ln2_b, DW.w1, W.b1, DW.w2, W.b2, dec_conv_of(c, l),
                                dec_ssm_of(c, l)};
    }
    p.L = D.L; p.r = D.r; p.lanes = lanes; p.maxlen = maxlen; p.ld_state = c->ld_dec;
    p.ln_n = D.dn;
    p.emb = c->emb; p.hw1 = c->dhw1; p.hb1 = c->hb1; p.hw2 = c->dhw2; p.hb2 = c->hb2;
    p.inv_t = c->inv_temp; p.tok = c->tok; p.lens = c->lens; p.t_counter = c->t_counter;
    p.out = out; p.out_stride = chunk; p.states = c->dec; p.payload = d_payload;
    p.offsets = c->offsets; p.sizes = c->sizes;
    return timed(c, BOA_K_DECODE, 1024.0 * lanes * (maxlen - 1),
                 [&] { return launch_dec_persist(p, D.d, D.ds, c->n_cus, s); });
  }
  // fp32 from 2048 lanes on: head.2 runs fused with the coder step
  // (dec_head_step_kernel), so the logits stay on chip; below that, and in
  // bf16, head.2 and the coder step are separate launches
  const bool fuse_head = !c->bf16 && dec_fuse_head(lanes);
  auto one_step = [&](hipStream_t gs) -> hipError_t {
    hipError_t e =
        step_range(c, 0, lanes, gs, c->t_counter, c->tok, false, c->dlogits, !fuse_head);
    if (e) return e;
    hipStream_t saved = c->stream;
    c->stream = gs;
    if (fuse_head) {
      DecGemmArgs h{};
      h.Xt = c->dot; h.ldx = c->ld_dec; h.W = c->dhw2; h.ldw = VOCAB; h.M = lanes; h.N = VOCAB;
      h.K = D.d; h.act = ACT_NONE; h.row_major = 1;
      e = timed(c, BOA_K_DECODE, 2.0 * lanes * VOCAB * D.d, [&] {
        return launch_dec_head_step(h, c->hb2, c->inv_temp, c->tok, c->lens, c->t_counter, out,
                                    chunk, c->dec, d_payload, c->offsets, c->sizes, gs);
      });
    } else {
      e = timed(c, BOA_K_DECODE, 1024.0 * lanes, [&] {
        return launch_decode_step(c->dlogits, c->hb2, c->inv_temp, c->tok, c->lens, c->t_counter,
                                  out, chunk, c->dec, d_payload, c->offsets, c->sizes, lanes, gs);
      });
    }
    c->stream = saved;
    return e;
  };
  // progress: every kProgSteps steps, once the steps before have run
  constexpr int kProgSteps = 2048;
  int64_t pend = -1;
  int slot = 0;
  const int64_t total = c->prog_total, base = c->prog_base;
  if (c->prof_on || maxlen <= 2) {
    for (int t = 1; t < maxlen; ++t) {
      hipError_t e = one_step(s);
      if (!e && c->progress && t % kProgSteps == 0)
        e = progress_mark(c, 1, base + (int64_t)lanes * (t + 1), total, &pend, &slot);
      if (e) return e;
    }
    return hipSuccess;
  }
  hipError_t e = hipSuccess;
  if (!c->dec_stream) e = hipStreamCreateWithFlags(&c->dec_stream, hipStreamNonBlocking);
  if (!e && !c->dec_fork) e = hipEventCreateWithFlags(&c->dec_fork, hipEventDisableTiming);
  if (!e && !c->dec_join) e = hipEventCreateWithFlags(&c->dec_join, hipEventDisableTiming);
  if (!e) e = hipEventRecord(c->dec_fork, s);
  if (!e) e = hipStreamWaitEvent(c->dec_stream, c->dec_fork, 0);
  if (e) return e;
  // the step's launch arguments; the executable graph is reused while they
  // stay the same (every pointer the step reads or writes is either one of
  // these or a buffer of the context)
  boa_ctx::GraphKey key;
  key.lanes = lanes; key.out = out; key.stride = chunk; key.payload = d_payload;
  key.inv_temp = c->inv_temp; key.stream = c->dec_stream;
  const boa_ctx::GraphKey& k0 = c->dec_key;
  const bool same = c->dec_exec && k0.lanes == key.lanes && k0.out == key.out &&
                    k0.stride == key.stride && k0.payload == key.payload &&
                    k0.inv_temp == key.inv_temp && k0.stream == key.stream;
  if (!same) {
    if (c->dec_exec) {
      e = hipStreamSynchronize(c->dec_stream);  // its last replay has finished
      (void)hipGraphExecDestroy(c->dec_exec);
      c->dec_exec = nullptr;
      if (e) return e;
    }
    hipGraph_t graph = nullptr;
    e = hipStreamBeginCapture(c->dec_stream, hipStreamCaptureModeThreadLocal);
    if (!e) {
      hipError_t le = one_step(c->dec_stream);
      e = hipStreamEndCapture(c->dec_stream, &graph);
      if (!e) e = le;
    }
    if (!e) e = hipGraphInstantiate(&c->dec_exec, graph, nullptr, nullptr, 0);
    if (graph) (void)hipGraphDestroy(graph);
    if (e) {
      c->dec_exec = nullptr;
      return e;
    }
    c->dec_key = key;
  }
  hipStream_t saved = c->stream;
  c->stream = c->dec_stream;  // progress markers go on the replay stream
  for (int t = 1; t < maxlen && !e; ++t) {
    e = hipGraphLaunch(c->dec_exec, c->dec_stream);
    if (!e && c->progress && t % kProgSteps == 0)
      e = progress_mark(c, 1, base + (int64_t)lanes * (t + 1), total, &pend, &slot);
  }
  c->stream = saved;
  hipError_t e2 = hipEventRecord(c->dec_join, c->dec_stream);
  if (!e2) e2 = hipStreamWaitEvent(s, c->dec_join, 0);
  return e ? e : e2;
}

}  // namespace

// ================================================================ C ABI
extern "C" {

int64_t boa_weight_file_bytes(int32_t d, int32_t L, int32_t ds, int32_t fp16) {
  const int64_t di = 2 * (int64_t)d, r = (d + 15) / 16, R = r + 2 * (int64_t)ds;
  const int64_t per_layer = 2 * d + 2 * di * d + 2 * di + di * 4 + di + R * di + di * r + di +
                            di * ds + di + d * di + d + 2 * d + 4 * (int64_t)d * d + 4 * d +
                            4 * (int64_t)d * d + d;
  const int64_t elems = 256 * (int64_t)d + L * per_layer + (int64_t)d * d + d + 256 * (int64_t)d + 256;
  return 4 + elems * (fp16 ? 2 : 4);
}

int boa_create(const boa_config* cfg, boa_ctx** out) {
  if (!cfg || !out) return BOA_E_ARG;
  *out = nullptr;
  const int d = cfg->d_model;
  // any d_model up to 512 (dt_rank = ceil(d / 16) <= 32): the kernels are
  // built for widths 64, 80 (the reference's ..._mambav1_80_1_20.pt), 128,
  // 256 and 512, and other widths run at the next one up (make_dims)
  if (d < 1 || d > 512 || cfg->n_layers < 1 || (cfg->d_state != 16 && cfg->d_state != 32) ||
      cfg->max_lanes < 1 || cfg->max_lanes > 65535 ||
      (cfg->precision != 0 && cfg->precision != 1) || cfg->tile < 0)
    return BOA_E_ARG;
  boa_ctx* c = new boa_ctx();
  {
    int dev = 0;
    if (hipGetDevice(&dev) != hipSuccess) { delete c; return BOA_E_HIP; }
    std::lock_guard<std::mutex> lock(g_scratch_mu);
    if (dev >= 0 && dev < kScratchDevices) {
      if (!g_scratch_ptr[dev]) {
        void* p = nullptr;
        if (hipGetSymbolAddress(&p, HIP_SYMBOL(scratch)) != hipSuccess || !p) {
          delete c;
          return BOA_E_HIP;
        }
        g_scratch_ptr[dev] = p;
      }
      c->scratch = (unsigned char*)g_scratch_ptr[dev];
    }
  }
  c->cfg = *cfg;
  if (!(c->cfg.temperature > 0.0f)) c->cfg.temperature = 1.0f;
  c->inv_temp = 1.0f / c->cfg.temperature;
  c->D = make_dims(*cfg);
  hipError_t e = hipStreamCreateWithFlags(&c->own_stream, hipStreamNonBlocking);
  if (e != hipSuccess) { delete c; return BOA_E_HIP; }
  c->stream = c->own_stream;
  const Dims& D = c->D;
  const size_t L = D.L, B = cfg->max_lanes;
  c->bf16 = cfg->precision == 1;
  c->ld_dec = (int)round_up(cfg->max_lanes, 64);
  c->n_xdec = dec_rb(D.r) + 2 * D.ds;
  const size_t ldd = c->ld_dec;
  if (dalloc(&c->dec_conv, L * D.di * ldd * 4) || dalloc(&c->dec_ssm, L * D.di * D.ds * ldd) ||
      dalloc(&c->dxt, D.d * ldd) || dalloc(&c->dxnt, D.d * ldd) || dalloc(&c->dot, D.d * ldd) ||
      dalloc(&c->dzt, D.di * ldd) || dalloc(&c->dcvt, D.di * ldd) || dalloc(&c->ddeltat, round_up(dec_rb(D.r) + 2 * D.ds, 16) * ldd) ||
      dalloc(&c->dyt, D.di * ldd) || dalloc(&c->dhidt, 4 * D.d * ldd) ||
      dalloc(&c->dlogits, B * VOCAB)) {
    boa_destroy(c);
    return BOA_E_NOMEM;
  }
  if (dalloc(&c->conv_state, L * B * D.di * 4) || dalloc(&c->ssm_state, L * B * D.di * D.ds) ||
      dalloc(&c->enc, B) || dalloc(&c->dec, B) || dalloc(&c->sizes, B) || dalloc(&c->offsets, B) ||
      dalloc(&c->lens, B) || dalloc(&c->tok, B) || dalloc(&c->t_counter, 1) ||
      hipHostMalloc((void**)&c->h_sizes, sizeof(int32_t) * B) != hipSuccess) {
    boa_destroy(c);
    return BOA_E_NOMEM;
  }
  {
    int dev = 0;
    if (hipGetDevice(&dev) != hipSuccess ||
        hipDeviceGetAttribute(&c->n_cus, hipDeviceAttributeMultiprocessorCount, dev) != hipSuccess)
      c->n_cus = 0;
  }
  *out = c;
  return BOA_OK;
}

void boa_destroy(boa_ctx* c) {
  if (!c) return;
  if (c->stream) (void)hipStreamSynchronize(c->stream);
  prof_flush(c);
  for (hipEvent_t e : c->ev_pool) (void)hipEventDestroy(e);
  dfree(c->wbuf); dfree(c->dwbuf); dfree(c->b16buf);
  dfree(c->conv_state); dfree(c->ssm_state);
  dfree(c->dec_conv); dfree(c->dec_ssm);
  dfree(c->dxt); dfree(c->dxnt); dfree(c->dot); dfree(c->dzt); dfree(c->dcvt); dfree(c->ddeltat);
  dfree(c->dyt); dfree(c->dhidt); dfree(c->dlogits);
  dfree(c->x); dfree(c->xn); dfree(c->xz); dfree(c->cv); dfree(c->delta); dfree(c->y);
  if (c->enc_stream) (void)hipStreamSynchronize(c->enc_stream);
  dfree(c->hid); dfree(c->lowprob); dfree(c->lowprob_alt);
  dfree(c->words); dfree(c->enc); dfree(c->dec); dfree(c->sizes); dfree(c->offsets);
  dfree(c->lens); dfree(c->tok); dfree(c->t_counter);
  if (c->h_sizes) (void)hipHostFree(c->h_sizes);
  drop_dec_graph(c);
  dfree(c->first_buf); dfree(c->reorder_words); dfree(c->reorder_off); dfree(c->reorder_sz);
  for (hipEvent_t e : c->prog_ev)
    if (e) (void)hipEventDestroy(e);
  if (c->dec_stream) (void)hipStreamDestroy(c->dec_stream);
  if (c->enc_stream) (void)hipStreamDestroy(c->enc_stream);
  for (hipEvent_t e : {c->lp_ready[0], c->lp_ready[1], c->lp_free[0], c->lp_free[1], c->enc_done})
    if (e) (void)hipEventDestroy(e);
  if (c->dec_fork) (void)hipEventDestroy(c->dec_fork);
  if (c->dec_join) (void)hipEventDestroy(c->dec_join);
  if (c->own_stream) (void)hipStreamDestroy(c->own_stream);
  delete c;
}

const char* boa_last_error(const boa_ctx* c) { return c ? c->err.c_str() : "null context"; }

int boa_set_stream(boa_ctx* c, void* s) {
  if (!c) return BOA_E_ARG;
  c->stream = (hipStream_t)s;
  return BOA_OK;
}

int boa_use_own_stream(boa_ctx* c) {
  if (!c) return BOA_E_ARG;
  c->stream = c->own_stream;
  return BOA_OK;
}

int boa_set_temperature(boa_ctx* c, float t) {
  if (!c || !(t > 0.0f)) return BOA_E_ARG;
  c->cfg.temperature = t;
  c->inv_temp = 1.0f / t;
  return BOA_OK;
}

int boa_set_progress(boa_ctx* c, boa_progress_fn fn, void* user) {
  if (!c) return BOA_E_ARG;
  c->progress = fn;
  c->progress_user = user;
  return BOA_OK;
}

int boa_set_state_cache_budget(boa_ctx* c, int64_t bytes) {
  if (!c) return BOA_E_ARG;
  drop_dec_graph(c);
  c->state_cache_budget = bytes < 0 ? -1 : bytes;
  return BOA_OK;
}

int boa_decode_plan(const boa_ctx* c, int32_t lanes, int32_t* cached_layers, int32_t* flags) {
  if (!c || lanes < 1 || lanes > c->cfg.max_lanes) return BOA_E_ARG;
  const Dims& D = c->D;
  const bool pers = !c->bf16 && dec_persist_fits(D.d, D.ds, D.r, D.L);
  const bool chain32 = !pers && !c->bf16;
  if (cached_layers) *cached_layers = pers ? D.L : dec_cached_layers(c, lanes);
  if (flags)
    *flags = (chain32 && dec_fuse_ln(c, lanes) ? BOA_PLAN_FUSED_LN : 0) |
             (pers ? BOA_PLAN_PERSISTENT : 0) |
             (chain32 && dec_fuse_xproj(c, lanes) ? BOA_PLAN_FUSED_XPROJ : 0) |
             (chain32 && dec_fuse_head(lanes) ? BOA_PLAN_FUSED_HEAD : 0);
  return BOA_OK;
}

int boa_set_warm_start(boa_ctx* c, int32_t interleave_batch) {
  if (!c || interleave_batch < 0) return BOA_E_ARG;
  c->warm_batch = interleave_batch;
  return BOA_OK;
}

int boa_load_weights_mem(boa_ctx* c, const void* data, size_t n) {
  if (!c || !data) return BOA_E_ARG;
  const Dims& D = c->D;
  const uint8_t* p = (const uint8_t*)data;
  HostReader rd{p, n, 0, false, false};
  // boa_gpu.hpp:994-1006: "BOA" + 0x01 is fp16, "BOA" + other byte is fp32,
  // anything else is a headerless fp32 file.
  const bool hdr = n >= 4 && p[0] == 'B' && p[1] == 'O' && p[2] == 'A';
  if (hdr) { rd.fp16 = p[3] == 0x01; rd.pos = 4; }
  const int64_t expect = boa_weight_file_bytes(D.dn, D.L, D.ds, rd.fp16) - (hdr ? 0 : 4);
  if ((int64_t)n != expect) {
    char msg[256];
    snprintf(msg, sizeof msg,
             "weight file has %zu bytes, expected %lld for d_model=%d n_layers=%d d_state=%d", n,
             (long long)expect, D.dn, D.L, D.ds);
    return fail(c, BOA_E_FORMAT, msg);
  }
  // device layout: Linear weights transposed to [in][ld] with ld a multiple
  // of 256 (zero padded) so every GEMM tile load stays in bounds.  A model
  // of d_model dn below the kernel width d (Dims) is placed into the width-d
  // layout: its features sit at 0 .. dn-1 (inner channels at 0 .. 2 dn-1 of
  // each half of in_proj's output), every other weight and bias is zero.
  const int dn = D.dn, din = 2 * D.dn;
  std::vector<std::pair<size_t, std::vector<float>>> parts;  // (offset floats, data)
  size_t total = 0;
  auto place = [&](std::vector<float>&& v) -> size_t {
    size_t off = total;
    total += round_up((int64_t)v.size(), 64);
    parts.emplace_back(off, std::move(v));
    return off;
  };
  auto same = [](int i) { return i; };
  auto xz_row = [&](int i) { return i < din ? i : i - din + D.di; };  // in_proj's two halves
  // a [rows][cols] Linear weight of the file -> [cols_pad][ld], output feature
  // i at column row_at(i)
  auto linear_t = [&](int rows, int cols, int cols_pad, int ld, auto row_at) -> size_t {
    std::vector<float> w;
    rd.vec(w, (size_t)rows * cols);
    std::vector<float> t((size_t)cols_pad * ld, 0.0f);
    if (!rd.bad)
      for (int i = 0; i < rows; ++i)
        for (int j = 0; j < cols; ++j) t[(size_t)j * ld + row_at(i)] = w[(size_t)i * cols + j];
    return place(std::move(t));
  };
  // `count` groups of `width` floats of the file -> groups at at(i) of
  // `count_pad` groups
  auto raw_at = [&](int count, int count_pad, int width, auto at) -> size_t {
    std::vector<float> v;
    rd.vec(v, (size_t)count * width);
    std::vector<float> t((size_t)count_pad * width, 0.0f);
    if (!rd.bad)
      for (int i = 0; i < count; ++i)
        memcpy(t.data() + (size_t)at(i) * width, v.data() + (size_t)i * width, 4 * (size_t)width);
    return place(std::move(t));
  };
  auto raw = [&](int count, int count_pad) -> size_t { return raw_at(count, count_pad, 1, same); };
  struct LayerOff {
    size_t ln1_w, ln1_b, w_in, b_in, conv_w, conv_b, w_x, w_dt, b_dt, a_log, na2, dd, w_out, b_out,
        ln2_w, ln2_b, w1, b1, w2, b2;
  };
  std::vector<LayerOff> lo(D.L);
  size_t emb;
  {  // embedding [256][dn] -> [256][d]
    std::vector<float> v;
    rd.vec(v, (size_t)VOCAB * dn);
    std::vector<float> t((size_t)VOCAB * D.d, 0.0f);
    if (!rd.bad)
      for (int i = 0; i < VOCAB; ++i)
        memcpy(t.data() + (size_t)i * D.d, v.data() + (size_t)i * dn, 4 * (size_t)dn);
    emb = place(std::move(t));
  }
  for (int l = 0; l < D.L; ++l) {
    LayerOff& o = lo[l];
    o.ln1_w = raw(dn, D.d);
    o.ln1_b = raw(dn, D.d);
    o.w_in = linear_t(2 * din, dn, D.d, D.ld_in, xz_row);
    o.b_in = raw_at(2 * din, 2 * D.di, 1, xz_row);
    o.conv_w = raw_at(din, D.di, 4, same);
    o.conv_b = raw(din, D.di);
    o.w_x = linear_t(D.R, din, D.di, D.ld_x, same);
    {  // dt_proj [di][r] stored as [r][di] (no padding: read per channel)
      std::vector<float> w;
      rd.vec(w, (size_t)din * D.r);
      std::vector<float> t((size_t)D.r * D.di, 0.0f);
      if (!rd.bad)
        for (int i = 0; i < din; ++i)
          for (int j = 0; j < D.r; ++j) t[(size_t)j * D.di + i] = w[(size_t)i * D.r + j];
      o.w_dt = place(std::move(t));
    }
    o.b_dt = raw(din, D.di);
    o.a_log = raw_at(din, D.di, D.ds, same);
    o.na2 = place(std::vector<float>((size_t)D.di * D.ds, 0.0f));
    o.dd = raw(din, D.di);
    o.w_out = linear_t(dn, din, D.di, D.ld_out, same);
    o.b_out = raw(dn, D.d);
    o.ln2_w = raw(dn, D.d);
    o.ln2_b = raw(dn, D.d);
    o.w1 = linear_t(4 * dn, dn, D.d, D.ld_1, same);
    o.b1 = raw(4 * dn, 4 * D.d);
    o.w2 = linear_t(dn, 4 * dn, 4 * D.d, D.ld_2, same);
    o.b2 = raw(dn, D.d);
  }
  const size_t hw1 = linear_t(dn, dn, D.d, D.ld_h1, same);
  const size_t hb1 = raw(dn, D.d);
  const size_t hw2 = linear_t(VOCAB, dn, D.d, D.ld_h2, same);
  const size_t hb2 = raw(VOCAB, VOCAB);
  if (rd.bad || rd.pos != n) return fail(c, BOA_E_FORMAT, "weight file truncated");

  drop_dec_graph(c);
  dfree(c->wbuf);
  c->wbuf = nullptr;
  c->loaded = false;
  if (dalloc(&c->wbuf, total)) return fail(c, BOA_E_NOMEM, "device allocation of weights failed");
  for (auto& pr : parts)
    if (!pr.second.empty())
      HIP_TRY(c, hipMemcpyAsync(c->wbuf + pr.first, pr.second.data(), pr.second.size() * 4,
                                hipMemcpyHostToDevice, c->stream));
  float* w = c->wbuf;
  c->emb = w + emb;
  c->hw1 = w + hw1; c->hb1 = w + hb1; c->hw2 = w + hw2; c->hb2 = w + hb2;
  c->layers.resize(D.L);
  for (int l = 0; l < D.L; ++l) {
    const LayerOff& o = lo[l];
    LayerW& L = c->layers[l];
    L.ln1_w = w + o.ln1_w; L.ln1_b = w + o.ln1_b; L.w_in = w + o.w_in; L.b_in = w + o.b_in;
    L.conv_w = w + o.conv_w; L.conv_b = w + o.conv_b; L.w_x = w + o.w_x; L.w_dt = w + o.w_dt;
    L.b_dt = w + o.b_dt; L.na2 = w + o.na2; L.dd = w + o.dd; L.w_out = w + o.w_out;
    L.b_out = w + o.b_out; L.ln2_w = w + o.ln2_w; L.ln2_b = w + o.ln2_b; L.w1 = w + o.w1;
    L.b1 = w + o.b1; L.w2 = w + o.w2; L.b2 = w + o.b2;
    // -exp(A_log) log2(e) once per load (mamba_kernels.cu:430-437), on the device so
    // that it is the same exp the kernels use.
    const int nA = D.di * D.ds;
    BOA_LAUNCH(na2_kernel, dim3((nA + 255) / 256), dim3(256), 0, c->stream,
                       w + o.a_log, w + o.na2, nA);
    HIP_TRY(c, hipGetLastError());
  }
  // k-blocked copies of the Linear weights for the decode step; x_proj's
  // copy inserts zero columns so that B starts at feature dec_rb(r)
  struct DecPart {
    const float* src;
    int ldw_in, n_src, K, N, permute, zs, ze;
    const float** dst;
  };
  std::vector<DecPart> dp;
  const int rb = dec_rb(D.r);
  c->dlayers.assign(D.L, boa_ctx::DecW{});
  for (int l = 0; l < D.L; ++l) {
    const LayerW& L = c->layers[l];
    boa_ctx::DecW& DW = c->dlayers[l];
    dp.push_back({L.w_in, D.ld_in, 2 * D.di, D.d, 2 * D.di, 1, 0, 0, &DW.w_in});
    dp.push_back({L.w_x, D.ld_x, D.R, D.di, c->n_xdec, 1, D.r, rb, &DW.w_x});
    dp.push_back({L.w_out, D.ld_out, D.d, D.di, D.d, 1, 0, 0, &DW.w_out});
    dp.push_back({L.w1, D.ld_1, 4 * D.d, D.d, 4 * D.d, 1, 0, 0, &DW.w1});
    dp.push_back({L.w2, D.ld_2, D.d, 4 * D.d, D.d, 1, 0, 0, &DW.w2});
  }
  dp.push_back({c->hw1, D.ld_h1, D.d, D.d, D.d, 1, 0, 0, &c->dhw1});
  dp.push_back({c->hw2, D.ld_h2, VOCAB, D.d, VOCAB, 0, 0, 0, &c->dhw2});
  size_t dtotal = 0;
  std::vector<size_t> doff;
  for (const DecPart& q : dp) {
    doff.push_back(dtotal);
    dtotal += (size_t)q.K * round_up(q.N, 16);
  }
  const size_t wdt_off = dtotal;
  dtotal += (size_t)D.L * D.di * (rb + D.ds);
  dfree(c->dwbuf);
  c->dwbuf = nullptr;
  if (dalloc(&c->dwbuf, dtotal)) return fail(c, BOA_E_NOMEM, "device allocation of weights failed");
  for (size_t i = 0; i < dp.size(); ++i) {
    const DecPart& q = dp[i];
    HIP_TRY(c, launch_dec_weight_blk(q.src, q.ldw_in, q.n_src, c->dwbuf + doff[i], q.K,
                                     (int)round_up(q.N, 16), q.permute, q.zs, q.ze, c->stream));
    *q.dst = c->dwbuf + doff[i];
  }
  for (int l = 0; l < D.L; ++l) {
    float* wq = c->dwbuf + wdt_off + (size_t)l * D.di * (rb + D.ds);
    float* nq = wq + (size_t)D.di * rb;
    HIP_TRY(c, launch_dec_scan_params(c->layers[l].w_dt, c->layers[l].na2, wq, nq, D.r, rb,
                                      D.ds, D.di, c->stream));
    c->dlayers[l].w_dt = wq;
    c->dlayers[l].na = nq;
  }
  if (c->bf16) {  // bf16 copies of the Linear weights: compress [N_pad][K], decode 32-blocked
    struct B16Part {
      const float* src;
      int ldw_in, n_src, K, N, zs, ze;
      const uint16_t** cdst;
      const uint16_t** ddst;
    };
    std::vector<B16Part> bp;
    c->b16c.assign(D.L, boa_ctx::B16W{});
    c->b16d.assign(D.L, boa_ctx::B16W{});
    for (int l = 0; l < D.L; ++l) {
      const LayerW& L = c->layers[l];
      boa_ctx::B16W &C_ = c->b16c[l], &D_ = c->b16d[l];
      bp.push_back({L.w_in, D.ld_in, 2 * D.di, D.d, 2 * D.di, 0, 0, &C_.w_in, &D_.w_in});
      bp.push_back({L.w_x, D.ld_x, D.R, D.di, D.R, 0, 0, &C_.w_x, nullptr});
      bp.push_back({L.w_x, D.ld_x, D.R, D.di, c->n_xdec, D.r, rb, nullptr, &D_.w_x});
      bp.push_back({L.w_out, D.ld_out, D.d, D.di, D.d, 0, 0, &C_.w_out, &D_.w_out});
      bp.push_back({L.w1, D.ld_1, 4 * D.d, D.d, 4 * D.d, 0, 0, &C_.w1, &D_.w1});
      bp.push_back({L.w2, D.ld_2, D.d, 4 * D.d, D.d, 0, 0, &C_.w2, &D_.w2});
    }
    bp.push_back({c->hw1, D.ld_h1, D.d, D.d, D.d, 0, 0, &c->b16c_h1, &c->b16d_h1});
    bp.push_back({c->hw2, D.ld_h2, VOCAB, D.d, VOCAB, 0, 0, &c->b16c_h2, &c->b16d_h2});
    size_t btotal = 0;
    std::vector<size_t> coff(bp.size()), doff2(bp.size());
    for (size_t i = 0; i < bp.size(); ++i) {
      const B16Part& q = bp[i];
      coff[i] = btotal;
      if (q.cdst) btotal += (size_t)round_up(q.N, 256) * q.K;
      doff2[i] = btotal;
      if (q.ddst) btotal += (size_t)q.K * round_up(q.N, 16);
    }
    dfree(c->b16buf);
    c->b16buf = nullptr;
    if (dalloc(&c->b16buf, btotal)) return fail(c, BOA_E_NOMEM, "device allocation of weights failed");
    for (size_t i = 0; i < bp.size(); ++i) {
      const B16Part& q = bp[i];
      if (q.cdst) {
        HIP_TRY(c, launch_b16_weight_nk(q.src, q.ldw_in, q.n_src, q.K, (int)round_up(q.N, 256),
                                        c->b16buf + coff[i], c->stream));
        *q.cdst = c->b16buf + coff[i];
      }
      if (q.ddst) {
        HIP_TRY(c, launch_dec_b16_weight(q.src, q.ldw_in, q.n_src, c->b16buf + doff2[i], q.K,
                                         (int)round_up(q.N, 16), q.zs, q.ze, c->stream));
        *q.ddst = c->b16buf + doff2[i];
      }
    }
  }
  HIP_TRY(c, hipStreamSynchronize(c->stream));
  c->loaded = true;
  return BOA_OK;
}

int boa_load_weights(boa_ctx* c, const char* path) {
  if (!c || !path) return BOA_E_ARG;
  std::vector<uint8_t> buf;
  if (!boa_read_file(path, buf)) return fail(c, BOA_E_IO, std::string("cannot read ") + path);
  return boa_load_weights_mem(c, buf.data(), buf.size());
}

int64_t boa_estimate_memory(const boa_config* cfg, int64_t chunk, int32_t compress) {
  if (!cfg) return -1;
  Dims D = make_dims(*cfg);
  const int64_t B = cfg->max_lanes;
  // padded transposes plus the k-blocked decode copies, upper bound
  int64_t w = boa_weight_file_bytes(D.d, D.L, D.ds, 0) * 3;
  int64_t state = 4 * (int64_t)D.L * B * D.di * (4 + D.ds);
  int64_t rows = B;
  int64_t words = 0;
  if (compress) {
    boa_ctx tmp;
    tmp.cfg = *cfg;
    tmp.D = D;
    rows = B * auto_tile(&tmp, chunk, (int)B);
    words = 4 * pitch_words_for(chunk) * B;
  }
  return w + state + rows * row_bytes(D) + words + (compress ? 0 : B * chunk);
}

int boa_reset_state(boa_ctx* c, int32_t lanes) {
  if (!c || lanes < 0 || lanes > c->cfg.max_lanes) return BOA_E_ARG;
  // Every lane is cleared (as reset_cache does for the whole batch), in both
  // state layouts.
  const Dims& D = c->D;
  const size_t B = c->cfg.max_lanes, ldd = c->ld_dec, L = D.L;
  HIP_TRY(c, launch_fill_zero(c->conv_state, sizeof(float) * L * B * D.di * 4, c->stream));
  HIP_TRY(c, launch_fill_zero(c->ssm_state, sizeof(float) * L * B * D.di * D.ds, c->stream));
  HIP_TRY(c, launch_fill_zero(c->dec_conv, sizeof(float) * L * D.di * ldd * 4, c->stream));
  HIP_TRY(c, launch_fill_zero(c->dec_ssm, sizeof(float) * L * D.di * D.ds * ldd, c->stream));
  c->state_mode = 2;
  return BOA_OK;
}

int boa_forward_chunk(boa_ctx* c, const uint8_t* d_tokens, int32_t lanes, int32_t T,
                      float* d_logits) {
  int rc = check_ready(c);
  if (rc) return rc;
  if (!d_tokens || !d_logits || lanes < 1 || lanes > c->cfg.max_lanes || T < 1)
    return fail(c, BOA_E_ARG, "boa_forward_chunk: bad arguments");
  if ((rc = ensure_rows(c, (int64_t)lanes * T))) return rc;
  TokenSrc tok{d_tokens, T, (int64_t)lanes * T, T};
  HIP_TRY(c, forward_tile(c, tok, lanes, T, 0, d_logits));
  return BOA_OK;
}

// Rows (lanes x T) that the scratch array holds: the seven activation
// buffers of a forward (x, xn [d]; xz [2 di]; conv, y [di]; delta [R];
// hidden [4 d] floats per row), each slice aligned to 256 bytes.
static int64_t noalloc_max_rows(const Dims& D) {
  const int64_t per_row = 4 * (int64_t)(14 * D.d + D.R);
  return ((int64_t)kScratchBytes - 7 * 256) / per_row;
}

int boa_forward_chunk_noalloc(boa_ctx* c, const uint8_t* d_tokens, int32_t lanes, int32_t T,
                              float* d_logits) {
  int rc = check_ready(c);
  if (rc) return rc;
  if (!d_tokens || !d_logits || lanes < 1 || lanes > c->cfg.max_lanes || T < 1)
    return fail(c, BOA_E_ARG, "boa_forward_chunk_noalloc: bad arguments");
  if (!c->scratch) return fail(c, BOA_E_STATE, "boa_forward_chunk_noalloc: no scratch on this device");
  const Dims& D = c->D;
  const int64_t rows = (int64_t)lanes * T, max_rows = noalloc_max_rows(D);
  if (rows > max_rows) {
    char msg[200];
    snprintf(msg, sizeof msg,
             "boa_forward_chunk_noalloc: lanes x T = %lld rows exceeds the %lld rows its %zu-byte "
             "scratch holds at d_model %d",
             (long long)rows, (long long)max_rows, kScratchBytes, D.d);
    return fail(c, BOA_E_ARG, msg);
  }
  // carve the scratch into the activation buffers of this call
  unsigned char* at = c->scratch;
  auto take = [&](int64_t floats) {
    float* p = (float*)at;
    at += round_up(floats * 4, 256);
    return p;
  };
  float *x = take(rows * D.d), *xn = take(rows * D.d), *xz = take(rows * 2 * D.di),
        *cv = take(rows * D.di), *delta = take(rows * D.R), *y = take(rows * D.di),
        *hid = take(rows * 4 * D.d);
  // the context's own buffers step aside for the call; profiling (which
  // creates events) is off during it
  float* saved[7] = {c->x, c->xn, c->xz, c->cv, c->delta, c->y, c->hid};
  const bool prof = c->prof_on;
  c->x = x; c->xn = xn; c->xz = xz; c->cv = cv; c->delta = delta; c->y = y; c->hid = hid;
  c->prof_on = false;
  TokenSrc tok{d_tokens, T, rows, T};
  hipError_t e = forward_tile(c, tok, lanes, T, 0, d_logits);
  c->x = saved[0]; c->xn = saved[1]; c->xz = saved[2]; c->cv = saved[3]; c->delta = saved[4];
  c->y = saved[5]; c->hid = saved[6];
  c->prof_on = prof;
  if (e) return hip_fail(c, e, "boa_forward_chunk_noalloc");
  return BOA_OK;
}

int boa_step_batch(boa_ctx* c, const uint8_t* d_tokens, int32_t lanes, float* d_logits,
                   int32_t add_bias) {
  int rc = check_ready(c);
  if (rc) return rc;
  if (!d_tokens || !d_logits || lanes < 1 || lanes > c->cfg.max_lanes)
    return fail(c, BOA_E_ARG, "boa_step_batch: bad arguments");
  HIP_TRY(c, step_forward(c, d_tokens, lanes, add_bias != 0, d_logits));
  return BOA_OK;
}

int boa_cdf_from_logits(boa_ctx* c, const float* d_logits, const float* d_bias, int32_t rows,
                        uint32_t* d_qcdf) {
  if (!c || !d_logits || !d_qcdf || rows < 1) return BOA_E_ARG;
  HIP_TRY(c, launch_cdf_rows(d_logits, d_bias, c->inv_temp, rows, d_qcdf, c->stream));
  return BOA_OK;
}

int boa_cdf_from_probs(boa_ctx* c, const float* d_probs, int32_t rows, int32_t K,
                       uint32_t* d_qcdf) {
  if (!c || !d_probs || !d_qcdf || rows < 1 || K < 1 || K > 1024) return BOA_E_ARG;
  HIP_TRY(c, launch_cdf_probs(d_probs, rows, K, d_qcdf, c->stream));
  return BOA_OK;
}

int boa_rc_encode_cdf(boa_ctx* c, const uint32_t* d_cdf, const uint8_t* d_syms, int32_t n_sym,
                      int32_t lanes, uint32_t* d_words, int64_t pitch_words, int32_t* d_sizes) {
  if (!c || !d_cdf || !d_syms || !d_words || !d_sizes || n_sym < 0 || lanes < 1 ||
      pitch_words < 2 * (int64_t)n_sym + 4)
    return BOA_E_ARG;
  HIP_TRY(c, launch_rc_encode_cdf(d_cdf, d_syms, n_sym, lanes, d_words, pitch_words, d_sizes, c->stream));
  return BOA_OK;
}

int boa_rc_decode_cdf(boa_ctx* c, const uint32_t* d_cdf, int32_t n_sym, int32_t lanes,
                      const uint32_t* d_words, int64_t pitch_words, const int32_t* d_sizes,
                      uint8_t* d_syms) {
  if (!c || !d_cdf || !d_syms || !d_words || !d_sizes || n_sym < 0 || lanes < 1) return BOA_E_ARG;
  HIP_TRY(c, launch_rc_decode_cdf(d_cdf, n_sym, lanes, d_words, pitch_words, d_sizes, d_syms, c->stream));
  return BOA_OK;
}

int64_t boa_num_chunks(int64_t n, int64_t chunk, int32_t max_chunks) {
  if (chunk <= 0 || n < 0) return -1;
  int64_t nc = (n + chunk - 1) / chunk;
  if (max_chunks > 0 && nc > max_chunks) nc = max_chunks;
  return nc;
}

int64_t boa_payload_bound_words(int64_t n, int64_t chunk, int32_t max_chunks) {
  int64_t nc = boa_num_chunks(n, chunk, max_chunks);
  if (nc < 0) return -1;
  return nc * pitch_words_for(chunk);
}

// Lanes of one batch iteration.  Cold: chunks u0 .. u0+G-1.  Warm-start
// (boa.cpp:395-401, 414): unit u runs chunk u*S + i at iteration i, and the
// units whose chunk exists lead the group.
static int iter_lanes(bool warm, int64_t nc, int64_t S, int64_t u0, int G, int64_t i) {
  if (!warm) return G;
  const int64_t live = (nc - i + S - 1) / S - u0;  // units u with u*S + i < nc, minus u0
  return (int)std::max<int64_t>(0, std::min<int64_t>(G, live));
}

int boa_compress_device(boa_ctx* c, const uint8_t* d_data, int64_t n, int64_t chunk,
                        int32_t max_chunks, uint32_t* d_payload, int64_t payload_cap_words,
                        uint64_t* h_stream_bytes, uint8_t* h_first, int64_t* h_payload_words) {
  int rc = check_ready(c);
  if (rc) return rc;
  if (!d_data || !d_payload || !h_stream_bytes || !h_first || n < 0 || chunk < 1 ||
      chunk > (1 << 30))
    return fail(c, BOA_E_ARG, "boa_compress_device: bad arguments");
  const int64_t nc = boa_num_chunks(n, chunk, max_chunks);
  if (nc > INT32_MAX) return fail(c, BOA_E_ARG, "boa_compress_device: too many chunks");
  if (h_payload_words) *h_payload_words = 0;
  if (nc == 0) return BOA_OK;
  const int B = c->cfg.max_lanes;
  const int64_t pitch = pitch_words_for(chunk);
  // warm-start: W lanes of S consecutive chunks each (boa.cpp:310-319)
  const bool warm = c->warm_batch > 0;
  const int64_t W = warm ? std::min<int64_t>(c->warm_batch, nc) : 0;
  const int64_t S = warm ? (nc + W - 1) / W : 1;
  const int64_t units = warm ? W : nc;
  const int64_t T = auto_tile(c, chunk, (int)std::min<int64_t>(B, units));
  if ((rc = ensure_rows(c, (int64_t)B * T))) return rc;
  if ((rc = ensure_words(c, pitch))) return rc;
  if ((rc = ensure_enc_stream(c))) return rc;
  hipStream_t s = c->stream;
  if (ensure_buf(&c->first_buf, &c->first_cap, nc))
    return fail(c, BOA_E_NOMEM, "device allocation of the first-byte buffer failed");
  BOA_LAUNCH(gather_first_kernel, dim3((unsigned)((nc + 255) / 256)), dim3(256), 0, s,
                     d_data, chunk, n, (int)nc, c->first_buf);
  hipError_t e = hipGetLastError();
  if (!e) e = hipMemcpyAsync(h_first, c->first_buf, (size_t)nc, hipMemcpyDeviceToHost, s);
  if (!e) e = hipStreamSynchronize(s);
  if (e) return hip_fail(c, e, "first bytes");
  const int64_t processed = std::min<int64_t>(n, nc * chunk);
  int64_t done = 0;  // input bytes of finished batch iterations
  // warm-start: where each chunk's stream landed in the iteration-ordered payload
  std::vector<uint64_t> stage_off(warm ? (size_t)nc : 0);
  int64_t out_words = 0;
  // an error after coder launches were queued: let the coder stream drain
  // (its kernels read the caller's input and write the context's words)
  // before the caller can free or reuse those buffers
  auto fail_coding = [&](hipError_t err, const char* where) {
    (void)hipStreamSynchronize(c->enc_stream);
    return hip_fail(c, err, where);
  };
  for (int64_t u0 = 0; u0 < units; u0 += B) {
    const int G = (int)std::min<int64_t>(B, units - u0);
    for (int64_t i = 0; i < S; ++i) {
      const int lanes = iter_lanes(warm, nc, S, u0, G, i);
      if (lanes == 0) break;
      const int64_t c0 = warm ? u0 * S + i : u0;  // chunk of lane 0
      const TokenSrc tok{d_data + c0 * chunk, warm ? S * chunk : chunk, n - c0 * chunk, chunk};
      // warm-start keeps the state across a unit's chunks (boa.cpp:432-435)
      if (i == 0 && (rc = boa_reset_state(c, G))) return rc;
      e = launch_rc_enc_init(c->enc, lanes, s);
      if (e) return hip_fail(c, e, "rc init");
      int64_t pend = -1;
      int slot = 0;
      int k = 0;  // tile index: buffer k & 1
      for (int64_t t0 = 0; t0 < chunk; t0 += T, ++k) {
        const int Tt = (int)std::min<int64_t>(T, chunk - t0);
        // the coder of tile k - 2 has finished reading this tile's buffer
        if (k >= 2) e = hipStreamWaitEvent(s, c->lp_free[k & 1], 0);
        if (e) return fail_coding(e, "compress tile");
        e = forward_tile_cdf(c, tok, lanes, Tt, (int)t0);
        if (!e) e = hipEventRecord(c->lp_ready[k & 1], s);
        if (!e) e = hipStreamWaitEvent(c->enc_stream, c->lp_ready[k & 1], 0);
        if (!e)
          e = timed(c, BOA_K_CODER, 8.0 * lanes * Tt, [&] {
            return launch_rc_encode_tile(c->lowprob, tok, Tt, (int)t0, lanes, c->enc, c->words,
                                         pitch, c->enc_stream);
          });
        if (!e) e = hipEventRecord(c->lp_free[k & 1], c->enc_stream);
        std::swap(c->lowprob, c->lowprob_alt);
        if (!e && c->progress)
          e = progress_mark(c, 0, std::min(processed, done + (int64_t)lanes * (t0 + Tt)), processed,
                            &pend, &slot);
        if (e) return fail_coding(e, "compress tile");
      }
      e = hipEventRecord(c->enc_done, c->enc_stream);  // the batch's last tile is coded
      if (!e) e = hipStreamWaitEvent(s, c->enc_done, 0);
      if (!e) e = launch_rc_finish(c->enc, c->words, pitch, c->sizes, lanes, s);
      if (!e) e = hipMemcpyAsync(c->h_sizes, c->sizes, sizeof(int32_t) * lanes, hipMemcpyDeviceToHost, s);
      if (!e) e = hipStreamSynchronize(s);
      if (e) return fail_coding(e, "finish");
      int64_t batch_words = 0;
      for (int b = 0; b < lanes; ++b) batch_words += c->h_sizes[b];
      if (out_words + batch_words > payload_cap_words)
        return fail(c, BOA_E_ARG, "payload buffer too small");
      e = timed(c, BOA_K_CODER, 8.0 * batch_words, [&] {
        return launch_compact(c->words, pitch, c->sizes, lanes, c->offsets, d_payload + out_words, s);
      });
      if (!e) e = hipStreamSynchronize(s);
      if (e) return hip_fail(c, e, "compaction");
      int64_t at = out_words;
      for (int b = 0; b < lanes; ++b) {
        const int64_t ci = warm ? (u0 + b) * S + i : u0 + b;
        h_stream_bytes[ci] = 4ull * (uint64_t)c->h_sizes[b];
        if (warm) stage_off[(size_t)ci] = (uint64_t)at;
        at += c->h_sizes[b];
        done += std::min<int64_t>(chunk, n - ci * chunk);
      }
      out_words += batch_words;
      if (c->progress) c->progress(c->progress_user, 0, done, processed);
    }
  }
  if (warm && S > 1 && out_words > 0) {
    // the container stores streams in chunk order (boa.cpp:560-565)
    std::vector<uint64_t> dst_off((size_t)nc);
    std::vector<int32_t> sizes((size_t)nc);
    uint64_t at = 0;
    for (int64_t ci = 0; ci < nc; ++ci) {
      dst_off[(size_t)ci] = at;
      sizes[(size_t)ci] = (int32_t)(h_stream_bytes[ci] / 4);
      at += sizes[(size_t)ci];
    }
    if (ensure_buf(&c->reorder_words, &c->reorder_words_cap, out_words))
      return fail(c, BOA_E_NOMEM, "device allocation of the reorder buffer failed");
    if (nc > c->reorder_n_cap) {
      dfree(c->reorder_off); dfree(c->reorder_sz);
      c->reorder_off = nullptr; c->reorder_sz = nullptr; c->reorder_n_cap = 0;
      if (dalloc(&c->reorder_off, 2 * (size_t)nc) || dalloc(&c->reorder_sz, (size_t)nc))
        return fail(c, BOA_E_NOMEM, "device allocation of the reorder buffer failed");
      c->reorder_n_cap = nc;
    }
    uint32_t* tmp = c->reorder_words;
    uint64_t* d_off = c->reorder_off;
    int32_t* d_sz = c->reorder_sz;
    e = hipMemcpyAsync(d_off, stage_off.data(), 8 * (size_t)nc, hipMemcpyHostToDevice, s);
    if (!e) e = hipMemcpyAsync(d_off + nc, dst_off.data(), 8 * (size_t)nc, hipMemcpyHostToDevice, s);
    if (!e) e = hipMemcpyAsync(d_sz, sizes.data(), 4 * (size_t)nc, hipMemcpyHostToDevice, s);
    if (!e)
      e = timed(c, BOA_K_CODER, 8.0 * out_words, [&] {
        return launch_gather_streams(d_payload, d_off, d_off + nc, d_sz, nc, tmp, s);
      });
    if (!e) e = hipMemcpyAsync(d_payload, tmp, 4 * (size_t)out_words, hipMemcpyDeviceToDevice, s);
    if (!e) e = hipStreamSynchronize(s);
    if (e) return hip_fail(c, e, "warm-start reorder");
  }
  if (h_payload_words) *h_payload_words = out_words;
  return BOA_OK;
}

int boa_decompress_device(boa_ctx* c, const uint32_t* d_payload, const uint64_t* h_offsets_words,
                          const uint64_t* h_stream_bytes, const uint8_t* h_first, int32_t nc,
                          int64_t chunk, int64_t last_len, uint8_t* d_out) {
  int rc = check_ready(c);
  if (rc) return rc;
  if (!d_payload || !h_offsets_words || !h_stream_bytes || !h_first || !d_out || nc < 0 ||
      chunk < 1 || last_len < 0 || last_len > chunk)
    return fail(c, BOA_E_ARG, "boa_decompress_device: bad arguments");
  if (nc == 0) return BOA_OK;
  const int B = c->cfg.max_lanes;
  const bool warm = c->warm_batch > 0;
  const int64_t W = warm ? std::min<int64_t>(c->warm_batch, nc) : 0;
  const int64_t S = warm ? (nc + W - 1) / W : 1;
  const int64_t units = warm ? W : nc;
  hipStream_t s = c->stream;
  std::vector<uint64_t> offs(B);
  std::vector<int32_t> nw(B), lens(B);
  std::vector<uint8_t> first(B);
  if (ensure_buf(&c->first_buf, &c->first_cap, B))
    return fail(c, BOA_E_NOMEM, "device allocation of the first-byte buffer failed");
  uint8_t* d_first = c->first_buf;
  const int64_t pitch_bytes = pitch_words_for(chunk) * 4;
  c->prog_total = (nc - 1) * chunk + last_len;
  c->prog_base = 0;
  for (int64_t u0 = 0; u0 < units; u0 += B) {
    const int G = (int)std::min<int64_t>(B, units - u0);
    for (int64_t i = 0; i < S; ++i) {
      const int lanes = iter_lanes(warm, nc, S, u0, G, i);
      if (lanes == 0) break;
      int32_t maxlen = 0;
      for (int b = 0; b < lanes; ++b) {
        const int64_t ci = warm ? (u0 + b) * S + i : u0 + b;
        if ((int64_t)h_stream_bytes[ci] > pitch_bytes)
          return fail(c, BOA_E_FORMAT, "stream too large for the chunk length");
        offs[b] = h_offsets_words[ci];
        nw[b] = (int32_t)(h_stream_bytes[ci] / 4);
        lens[b] = (int32_t)(ci == nc - 1 ? last_len : chunk);
        first[b] = h_first[ci];
        maxlen = std::max(maxlen, lens[b]);
      }
      hipError_t e = hipMemcpyAsync(c->offsets, offs.data(), 8 * lanes, hipMemcpyHostToDevice, s);
      if (!e) e = hipMemcpyAsync(c->sizes, nw.data(), 4 * lanes, hipMemcpyHostToDevice, s);
      if (!e) e = hipMemcpyAsync(c->lens, lens.data(), 4 * lanes, hipMemcpyHostToDevice, s);
      if (!e) e = hipMemcpyAsync(d_first, first.data(), lanes, hipMemcpyHostToDevice, s);
      if (e) return hip_fail(c, e, "decode upload");
      // warm-start resets the state only before a unit's first chunk (boa.cpp:690-693)
      if (i == 0 && (rc = boa_reset_state(c, G))) return rc;
      const int64_t c0 = warm ? u0 * S + i : u0;
      const int64_t stride = warm ? S * chunk : chunk;
      uint8_t* out = d_out + c0 * chunk;
      BOA_LAUNCH(decode_init_kernel, dim3((lanes + 255) / 256), dim3(256), 0, s, d_first,
                         c->lens, c->tok, out, stride, lanes, c->t_counter);
      e = hipGetLastError();
      if (!e) e = launch_rc_dec_init(c->dec, d_payload, c->offsets, c->sizes, lanes, s);
      if (!e) e = ensure_state_layout(c, 1);
      if (e) return hip_fail(c, e, "decode init");
      e = decode_steps(c, lanes, maxlen, out, stride, d_payload);
      if (e) return hip_fail(c, e, "decode step");
      // The compressor's state consumed every byte of the chunk; the units
      // that go on feed the last decoded byte before their next chunk.
      const int next = warm && i + 1 < S ? iter_lanes(warm, nc, S, u0, G, i + 1) : 0;
      if (next > 0) {
        e = step_forward(c, c->tok, next, false, c->dlogits);
        if (e) return hip_fail(c, e, "warm-start carry step");
      }
      e = hipStreamSynchronize(s);
      if (e) return hip_fail(c, e, "decode sync");
      for (int b = 0; b < lanes; ++b) c->prog_base += lens[b];
      if (c->progress) c->progress(c->progress_user, 1, c->prog_base, c->prog_total);
    }
  }
  return BOA_OK;
}

int boa_compress_buffer(boa_ctx* c, const uint8_t* h_in, int64_t n, int64_t chunk,
                        int32_t max_chunks, uint8_t** h_out, int64_t* out_len) {
  int rc = check_ready(c);
  if (rc) return rc;
  if ((!h_in && n) || !h_out || !out_len || chunk < 1) return fail(c, BOA_E_ARG, "bad arguments");
  const int64_t nc = boa_num_chunks(n, chunk, max_chunks);
  const int64_t processed = std::min<int64_t>(n, nc * chunk);
  uint8_t* d_in = nullptr;
  uint32_t* d_pay = nullptr;
  const int64_t cap = std::max<int64_t>(boa_payload_bound_words(n, chunk, max_chunks), 1);
  if (dalloc(&d_in, (size_t)std::max<int64_t>(n, 1)) || dalloc(&d_pay, (size_t)cap)) {
    dfree(d_in);
    return fail(c, BOA_E_NOMEM, "allocation failed");
  }
  const double t0 = now_s();
  if (n) {
    hipError_t e = hipMemcpyAsync(d_in, h_in, (size_t)n, hipMemcpyHostToDevice, c->stream);
    if (!e) e = hipStreamSynchronize(c->stream);
    if (e) { dfree(d_in); dfree(d_pay); return hip_fail(c, e, "upload"); }
  }
  const double t1 = now_s();
  std::vector<uint64_t> lens((size_t)std::max<int64_t>(nc, 1));
  std::vector<uint8_t> first((size_t)std::max<int64_t>(nc, 1));
  int64_t words = 0;
  rc = boa_compress_device(c, d_in, n, chunk, max_chunks, d_pay, cap, lens.data(), first.data(), &words);
  if (rc) { dfree(d_in); dfree(d_pay); return rc; }
  const double t2 = now_s();
  std::vector<uint8_t> payload((size_t)words * 4);
  if (words) {
    hipError_t e = hipMemcpy(payload.data(), d_pay, (size_t)words * 4, hipMemcpyDeviceToHost);
    if (e) { dfree(d_in); dfree(d_pay); return hip_fail(c, e, "download"); }
  }
  c->t_h2d = t1 - t0;
  c->t_compute = t2 - t1;
  c->t_d2h = now_s() - t2;
  dfree(d_in);
  dfree(d_pay);
  Boa2Header h;
  h.total_size = (uint64_t)processed;
  h.chunk_len = (uint32_t)chunk;
  h.n_chunks = (uint32_t)nc;
  h.last_chunk_len = (uint32_t)(nc > 1 ? processed - (nc - 1) * chunk : processed);
  if (c->warm_batch > 0) {  // flags bit 0 + u32 interleave batch (boa.cpp:542-559)
    const uint32_t W = (uint32_t)std::min<int64_t>(c->warm_batch, nc);
    h.flags = 1u;
    h.fp.resize(4);
    memcpy(h.fp.data(), &W, 4);
  }
  std::vector<uint8_t> blob;
  boa2_write(h, payload, first.data(), lens.data(), (size_t)nc, blob);
  uint8_t* o = (uint8_t*)malloc(blob.size() ? blob.size() : 1);
  if (!o) return fail(c, BOA_E_NOMEM, "host allocation failed");
  memcpy(o, blob.data(), blob.size());
  *h_out = o;
  *out_len = (int64_t)blob.size();
  return BOA_OK;
}

int boa_decompress_buffer(boa_ctx* c, const uint8_t* h_in, int64_t n, uint8_t** h_out,
                          int64_t* out_len) {
  int rc = check_ready(c);
  if (rc) return rc;
  if (!h_in || !h_out || !out_len) return fail(c, BOA_E_ARG, "bad arguments");
  Boa2Parsed P;
  std::string why;
  if (!boa2_parse(h_in, (size_t)n, P, why)) return fail(c, BOA_E_FORMAT, why);
  const size_t nc = P.hdr.n_chunks;
  // warm-start: the interleave batch comes from the header (boa.cpp:603-610)
  const bool warm = (P.hdr.flags & 1u) != 0;
  if (warm && nc > 0 && P.interleave_batch == 0)
    return fail(c, BOA_E_FORMAT, "warm-start container without a valid interleave batch");
  if (nc == 0) {  // empty input
    *h_out = (uint8_t*)malloc(1);
    if (!*h_out) return fail(c, BOA_E_NOMEM, "host allocation failed");
    *out_len = 0;
    return BOA_OK;
  }
  // streams re-packed on 32-bit word boundaries
  std::vector<uint64_t> offs(std::max<size_t>(nc, 1)), lens(std::max<size_t>(nc, 1));
  uint64_t words = 0;
  for (size_t i = 0; i < nc; ++i) {
    offs[i] = words;
    lens[i] = P.lengths[i];
    words += (P.lengths[i] + 3) / 4;
  }
  std::vector<uint32_t> packed((size_t)std::max<uint64_t>(words, 1), 0u);
  for (size_t i = 0; i < nc; ++i)
    memcpy(packed.data() + offs[i], h_in + P.payload_off + P.offsets[i], P.lengths[i]);
  int64_t total = 0;
  for (size_t i = 0; i < nc; ++i) total += (i == nc - 1) ? P.hdr.last_chunk_len : P.hdr.chunk_len;
  uint32_t* d_pay = nullptr;
  uint8_t* d_out = nullptr;
  if (dalloc(&d_pay, packed.size()) || dalloc(&d_out, (size_t)std::max<int64_t>(total, 1))) {
    dfree(d_pay);
    return fail(c, BOA_E_NOMEM, "allocation failed");
  }
  const double t0 = now_s();
  hipError_t e = hipMemcpy(d_pay, packed.data(), packed.size() * 4, hipMemcpyHostToDevice);
  if (e) { dfree(d_pay); dfree(d_out); return hip_fail(c, e, "upload"); }
  const double t1 = now_s();
  const int32_t saved_warm = c->warm_batch;
  c->warm_batch = warm ? (int32_t)P.interleave_batch : 0;
  rc = boa_decompress_device(c, d_pay, offs.data(), lens.data(), P.first.data(), (int32_t)nc,
                             P.hdr.chunk_len, nc ? P.hdr.last_chunk_len : 0, d_out);
  c->warm_batch = saved_warm;
  if (rc) { dfree(d_pay); dfree(d_out); return rc; }
  const double t2 = now_s();
  uint8_t* o = (uint8_t*)malloc((size_t)std::max<int64_t>(total, 1));
  if (!o) { dfree(d_pay); dfree(d_out); return fail(c, BOA_E_NOMEM, "host allocation failed"); }
  if (total) e = hipMemcpy(o, d_out, (size_t)total, hipMemcpyDeviceToHost);
  c->t_h2d = t1 - t0;
  c->t_compute = t2 - t1;
  c->t_d2h = now_s() - t2;
  dfree(d_pay);
  dfree(d_out);
  if (e) { free(o); return hip_fail(c, e, "download"); }
  *h_out = o;
  *out_len = total;
  return BOA_OK;
}

int boa_compress_file(boa_ctx* c, const char* in_path, const char* out_path, int64_t chunk,
                      int32_t max_chunks) {
  if (!c || !in_path || !out_path) return BOA_E_ARG;
  std::vector<uint8_t> in;
  if (!boa_read_file(in_path, in)) return fail(c, BOA_E_IO, std::string("cannot read ") + in_path);
  uint8_t* out = nullptr;
  int64_t n = 0;
  int rc = boa_compress_buffer(c, in.data(), (int64_t)in.size(), chunk, max_chunks, &out, &n);
  if (rc) return rc;
  bool ok = boa_write_file(out_path, out, (size_t)n);
  free(out);
  return ok ? BOA_OK : fail(c, BOA_E_IO, std::string("cannot write ") + out_path);
}

int boa_decompress_file(boa_ctx* c, const char* in_path, const char* out_path) {
  if (!c || !in_path || !out_path) return BOA_E_ARG;
  std::vector<uint8_t> in;
  if (!boa_read_file(in_path, in)) return fail(c, BOA_E_IO, std::string("cannot read ") + in_path);
  uint8_t* out = nullptr;
  int64_t n = 0;
  int rc = boa_decompress_buffer(c, in.data(), (int64_t)in.size(), &out, &n);
  if (rc) return rc;
  bool ok = boa_write_file(out_path, out, (size_t)n);
  free(out);
  return ok ? BOA_OK : fail(c, BOA_E_IO, std::string("cannot write ") + out_path);
}

void boa_free(void* p) { free(p); }

uint32_t boa_crc32(const uint8_t* data, int64_t n) { return boa2_crc32(data, (size_t)n); }

int boa_last_timings(const boa_ctx* c, double* h2d_s, double* compute_s, double* d2h_s) {
  if (!c) return BOA_E_ARG;
  if (h2d_s) *h2d_s = c->t_h2d;
  if (compute_s) *compute_s = c->t_compute;
  if (d2h_s) *d2h_s = c->t_d2h;
  return BOA_OK;
}

int boa_profile_enable(boa_ctx* c, int32_t on) {
  if (!c) return BOA_E_ARG;
  if (!on) prof_flush(c);
  c->prof_on = on != 0;
  return BOA_OK;
}

int boa_profile_reset(boa_ctx* c) {
  if (!c) return BOA_E_ARG;
  prof_flush(c);
  for (int k = 0; k < BOA_K_COUNT; ++k) { c->prof_ms[k] = 0; c->prof_work[k] = 0; c->prof_n[k] = 0; }
  return BOA_OK;
}

int boa_profile_read(boa_ctx* c, int32_t k, double* ms, int64_t* n, double* work) {
  if (!c || k < 0 || k >= BOA_K_COUNT) return BOA_E_ARG;
  prof_flush(c);
  if (ms) *ms = c->prof_ms[k];
  if (n) *n = c->prof_n[k];
  if (work) *work = c->prof_work[k];
  return BOA_OK;
}

}  // extern "C"
