// `boa` command-line driver over the C ABI (include/boa_hip.h).
//
// Same invocation as the reference driver (portability_solved_cpp/boa.cpp
// :819-942):
//   boa <compress|decompress> <model.bin> <input> <output> [d_model=256]
//       [n_layers=1] [--gpu-batch B] [--max-chunks C] [--chunk-size S]
//       [--tile T] [--temperature T] [--backbone mamba] [--show-timings]
//       [--no-graph] [--warm-start] [--d-state N] [--precision fp32|bf16]
//       [--kernel-timings]
// --show-timings prints the H2D / Compute / D2H phases (boa.cpp:504-507)
// of the unprofiled run.  --kernel-timings adds the summed kernel times of
// the model and of the coder from HIP events around every launch; such a
// run launches the decode steps directly instead of replaying their graph,
// so its throughput line is that of a profiled run.
// --gpu-batch 0 (default) sizes the batch from free device memory like
// auto_size_params (boa.cpp:109-156).  --warm-start interleaves chunks over
// the batch's lanes and carries state across them (boa.cpp:310-319); the
// decoder takes the interleave batch from the container.  --measure-energy
// is not provided.
#include <hip/hip_runtime.h>

#include <chrono>
#include <cstdint>
#include <cstdio>
#include <cstdlib>
#include <cstring>
#include <string>
#include <vector>

#include "../../include/boa_hip.h"

static int usage() {
  fprintf(stderr,
          "Usage: boa <compress|decompress> <model> <input> <output> [d_model] [n_layers] "
          "[--gpu-batch B] [--max-chunks C] [--chunk-size S] [--tile T] [--temperature T] "
          "[--warm-start] [--d-state N] [--precision fp32|bf16] [--show-timings] "
          "[--kernel-timings]\n");
  return 1;
}

// --gpu-batch 0: size the lane batch from free device memory, the steps of
// auto_size_params (boa.cpp:109-156): start at 64 (compress) or 1024
// (decompress) lanes, halve while the estimate exceeds 90 % of free memory,
// and if one lane still does not fit halve the chunk size down to 256 bytes;
// otherwise double while the next size fits, up to 8192 lanes.
static int auto_batch(boa_config cfg, int64_t& chunk, bool compress) {
  size_t free_b = 0, total_b = 0;
  if (hipMemGetInfo(&free_b, &total_b) != hipSuccess) return compress ? 64 : 1024;
  const int64_t target = (int64_t)(free_b * 0.9);
  int b = compress ? 64 : 1024;
  auto est = [&](int lanes) {
    cfg.max_lanes = lanes;
    return boa_estimate_memory(&cfg, chunk, compress);
  };
  int64_t mem = est(b);
  if (mem > target) {
    while (b > 1 && mem > target) {
      b /= 2;
      mem = est(b);
    }
    while (chunk > 256 && mem > target) {
      chunk /= 2;
      mem = est(b);
    }
  } else {
    while (b * 2 <= 8192 && est(b * 2) < target) b *= 2;
  }
  mem = est(b);
  printf("Auto-sizing: Selected Batch=%d, Chunk=%lld (%lld MB VRAM est, %lld MB free)\n", b,
         (long long)chunk, (long long)(mem >> 20), (long long)(free_b >> 20));
  return b;
}

// Progress bar in the form of print_progress (boa.cpp:30-50): percent of the
// input done and MB/s (2^20 B/s) so far.
struct Progress {
  std::chrono::steady_clock::time_point t0 = std::chrono::steady_clock::now();
  const char* prefix = "";
};

static void on_progress(void* user, int32_t, int64_t done, int64_t total) {
  const Progress* p = (const Progress*)user;
  const double sec =
      std::chrono::duration<double>(std::chrono::steady_clock::now() - p->t0).count();
  const double frac = total > 0 ? (double)done / (double)total : 1.0;
  const int width = 40, pos = (int)(width * frac);
  char bar[64];
  for (int i = 0; i < width; ++i) bar[i] = i < pos ? '=' : (i == pos ? '>' : ' ');
  bar[width] = 0;
  printf("\r%s [%s] %d%% %.2f MB/s", p->prefix, bar, (int)(frac * 100),
         sec > 0 ? (double)done / (1024.0 * 1024.0) / sec : 0.0);
  fflush(stdout);
}

int main(int argc, char** argv) {
  if (argc < 5) return usage();
  std::vector<std::string> args;
  int gpu_batch = 0, max_chunks = -1, tile = 0, d_state = 16, precision = 0;
  long long chunk = 4096;
  float temperature = 1.0f;
  bool show_timings = false, kernel_timings = false, warm_start = false;
  for (int i = 1; i < argc; ++i) {
    std::string s = argv[i];
    auto next = [&](const char* name) -> const char* {
      if (i + 1 >= argc) { fprintf(stderr, "missing value for %s\n", name); exit(1); }
      return argv[++i];
    };
    if (s == "--gpu-batch") gpu_batch = atoi(next("--gpu-batch"));
    else if (s == "--max-chunks") max_chunks = atoi(next("--max-chunks"));
    else if (s == "--chunk-size") chunk = atoll(next("--chunk-size"));
    else if (s == "--tile") tile = atoi(next("--tile"));
    else if (s == "--temperature") temperature = (float)atof(next("--temperature"));
    else if (s == "--d-state") d_state = atoi(next("--d-state"));
    else if (s == "--precision") {
      std::string p = next("--precision");
      if (p == "fp32") precision = 0;
      else if (p == "bf16") precision = 1;
      else { fprintf(stderr, "precision %s is not supported\n", p.c_str()); return 1; }
    } else if (s == "--backbone") {
      std::string b = next("--backbone");
      if (b != "mamba" && b != "mambav1") {
        fprintf(stderr, "backbone %s is not supported (mambav1 only)\n", b.c_str());
        return 1;
      }
    } else if (s == "--show-timings") show_timings = true;
    else if (s == "--kernel-timings") kernel_timings = true;
    else if (s == "--no-graph" || s == "--gpu") continue;
    else if (s == "--warm-start") warm_start = true;
    else if (s.rfind("--", 0) == 0) fprintf(stderr, "Warning: Unknown flag '%s' ignored.\n", s.c_str());
    else args.push_back(s);
  }
  if (args.size() < 4) return usage();
  const std::string mode = args[0], model = args[1], in = args[2], out = args[3];
  boa_config cfg{};
  cfg.d_model = args.size() > 4 ? atoi(args[4].c_str()) : 256;
  cfg.n_layers = args.size() > 5 ? atoi(args[5].c_str()) : 1;
  cfg.d_state = d_state;
  cfg.tile = tile;
  cfg.precision = precision;
  cfg.temperature = temperature;
  if (chunk <= 0) chunk = 4096;
  const bool compress = mode == "compress";
  if (!compress && mode != "decompress") { fprintf(stderr, "Unknown mode: %s\n", mode.c_str()); return 1; }
  int64_t chunk64 = chunk;
  cfg.max_lanes = gpu_batch > 0 ? gpu_batch : auto_batch(cfg, chunk64, compress);
  chunk = chunk64;
  boa_ctx* ctx = nullptr;
  int rc = boa_create(&cfg, &ctx);
  if (rc) { fprintf(stderr, "boa_create failed (%d)\n", rc); return 1; }
  rc = boa_load_weights(ctx, model.c_str());
  if (rc) { fprintf(stderr, "load weights: %s\n", boa_last_error(ctx)); boa_destroy(ctx); return 1; }
  if (compress && warm_start) {
    boa_set_warm_start(ctx, cfg.max_lanes);
    printf("Using warm-start interleaved compression. Batch=%d\n", cfg.max_lanes);
  }
  Progress prog;
  prog.prefix = compress ? "Compressing" : "Decompressing";
  boa_set_progress(ctx, on_progress, &prog);
  if (kernel_timings) boa_profile_enable(ctx, 1);
  auto t0 = std::chrono::steady_clock::now();
  prog.t0 = t0;
  rc = compress ? boa_compress_file(ctx, in.c_str(), out.c_str(), chunk, max_chunks)
                : boa_decompress_file(ctx, in.c_str(), out.c_str());
  double sec = std::chrono::duration<double>(std::chrono::steady_clock::now() - t0).count();
  if (rc) { fprintf(stderr, "\n%s failed: %s\n", mode.c_str(), boa_last_error(ctx)); boa_destroy(ctx); return 1; }
  FILE* f = fopen(compress ? in.c_str() : out.c_str(), "rb");
  long long nbytes = 0;
  if (f) { fseek(f, 0, SEEK_END); nbytes = ftell(f); fclose(f); }
  printf("\nDone. Time: %.3fs, Avg Throughput: %.3f MB/s%s\n", sec,
         nbytes / (1024.0 * 1024.0) / (sec > 0 ? sec : 1),
         kernel_timings ? " (profiled run: every launch timed)" : "");
  if (show_timings) {  // H2D / Compute / D2H as boa.cpp:504-507
    double h2d = 0, comp = 0, d2h = 0;
    boa_last_timings(ctx, &h2d, &comp, &d2h);
    printf("Timing (s): H2D=%.3f Compute=%.3f D2H=%.3f\n", h2d, comp, d2h);
  }
  if (kernel_timings) {
    // summed kernel times of the model (head.2 + CDF included where they run
    // fused) and of the CDF and coder kernels
    double fwd = 0, enc = 0;
    const int fwd_k[] = {BOA_K_GEMM, BOA_K_SCAN, BOA_K_CONV, BOA_K_LN, BOA_K_GEMM_SMALL,
                         BOA_K_DEC_GEMM, BOA_K_DEC_SCAN, BOA_K_HEAD_CDF, BOA_K_DEC_LNGEMM};
    const int enc_k[] = {BOA_K_CDF, BOA_K_CODER, BOA_K_DECODE};
    for (int k : fwd_k) { double ms = 0; boa_profile_read(ctx, k, &ms, nullptr, nullptr); fwd += ms * 1e-3; }
    for (int k : enc_k) { double ms = 0; boa_profile_read(ctx, k, &ms, nullptr, nullptr); enc += ms * 1e-3; }
    printf("Kernel time (s): Forward=%.3f Encode=%.3f\n", fwd, enc);
  }
  boa_destroy(ctx);
  return 0;
}
