/*
 * boa_hip.h -- C ABI of the MI355X-native BoaConstrictor codec path.
 *
 * Drop-in boundary for the chunk-parallel compress/decompress hot path of
 * the reference's C++ driver (portability_solved_cpp/boa.cpp, boa_gpu.hpp,
 * gemm_gpu.hpp).  The reference binds its kernels through C++ launchers at
 * single-op granularity (gemm_gpu.hpp:124-265); this ABI exports the same
 * capabilities at fused-op granularity with plain pointers, sizes and
 * integer status codes (no exit(), no C++ or torch types).
 *
 * Conventions
 *   - Every function returns BOA_OK (0) or a negative BOA_E* code; the
 *     message of the last failure is boa_last_error(ctx).
 *   - "d_" arguments are device pointers (hipMalloc'd or torch tensors),
 *     "h_" arguments are host pointers.
 *   - All work of a context is ordered on the context's HIP stream; a
 *     context is not thread-safe, separate contexts are independent.
 *   - Tokens and bytes are uint8; logits are fp32 [rows][256].
 */
#ifndef BOA_HIP_H
#define BOA_HIP_H

#include <stddef.h>
#include <stdint.h>

#ifdef __cplusplus
extern "C" {
#endif

#define BOA_OK 0
#define BOA_E_ARG -1      /* invalid argument / unsupported shape */
#define BOA_E_HIP -2      /* HIP runtime error */
#define BOA_E_IO -3       /* file read/write error */
#define BOA_E_FORMAT -4   /* malformed weight file or container */
#define BOA_E_STATE -5    /* call out of order (e.g. no weights loaded) */
#define BOA_E_NOMEM -6    /* device or host allocation failed */

typedef struct boa_ctx boa_ctx;

/* Model and batching configuration.
 * Replaces MambaConfig (gemm_gpu.hpp:38-66) plus the --gpu-batch / --tile /
 * --temperature CLI state of boa.cpp:838-897.  d_conv = 4 and expand = 2 are
 * fixed as in the reference; dt_rank = ceil(d_model / 16). */
typedef struct {
    int32_t d_model;     /* 1 .. 512.  The kernels are built for widths 64, 80,
                            128, 256 and 512 (bf16: 64, 128, 256, 512); another
                            d_model runs at the next built width with its extra
                            features zero, giving the d_model's own results */
    int32_t n_layers;
    int32_t d_state;     /* 16 or 32 (the reference supports 16 only) */
    int32_t max_lanes;   /* chunks processed in parallel (--gpu-batch) */
    int32_t tile;        /* compress forward tile in tokens (--tile); 0 = auto */
    int32_t precision;   /* 0 = fp32; 1 = bf16 weights and activations (fp32
                            accumulation, residual stream, scan state, logits) */
    float temperature;   /* softmax temperature (--temperature), 1.0 default */
} boa_config;

/* Context lifetime.  Replaces BoaPredictorGPU's constructor and free()
 * (boa_gpu.hpp:945-969, 1163-1173) and g_stream (gemm_gpu.hpp:111). */
int boa_create(const boa_config* cfg, boa_ctx** out);
void boa_destroy(boa_ctx* ctx);
const char* boa_last_error(const boa_ctx* ctx);
/* Order all later work on an external HIP stream (hipStream_t; NULL is the
 * null stream); boa_use_own_stream returns to the context's own stream. */
int boa_set_stream(boa_ctx* ctx, void* hip_stream);
int boa_use_own_stream(boa_ctx* ctx);
/* gpu_set_temperature (range_coder_kernels.cu:9-12). */
int boa_set_temperature(boa_ctx* ctx, float temperature);
/* Warm-start interleave (--warm-start; boa.cpp:310-319, 395-435, 690-693).
 * With interleave_batch B > 0, boa_compress_device / boa_decompress_device
 * run W = min(B, n_chunks) units of S = ceil(n_chunks / W) consecutive
 * chunks each, unit u taking chunks u*S + i, and carry the recurrent state
 * from one chunk of a unit to the next (reset only before the first).
 * Units are run max_lanes at a time.  Streams stay in chunk order.  The
 * buffer and file calls write flags bit 0 and W to the BOA2 header, and
 * take W from the header when reading (whatever this setting is).  The
 * decoder feeds each chunk's last byte before the unit's next chunk, as the
 * compressor's forward consumed it.  0 (default) = every chunk starts from
 * zero state. */
int boa_set_warm_start(boa_ctx* ctx, int32_t interleave_batch);

/* Progress reports, the callback form of print_progress (boa.cpp:30-50,
 * called per batch at :410 and :688).  fn(user, phase, done, total) is
 * called on the calling thread during boa_compress_* (phase 0) and
 * boa_decompress_* (phase 1) with input bytes done and the call's total:
 * per compress tile and batch, and every 2048 decode steps and per batch,
 * each report once the device has finished that work.  NULL turns the
 * reports off (the default); without a callback no synchronisation is
 * added. */
typedef void (*boa_progress_fn)(void* user, int32_t phase, int64_t done_bytes, int64_t total_bytes);
int boa_set_progress(boa_ctx* ctx, boa_progress_fn fn, void* user);

/* Decode-step plan (no reference counterpart; a diagnostic of this build's
 * schedule for `lanes` lanes): how many layers keep their recurrent state in
 * the caches (the rest stream it past them), and BOA_PLAN_* flags: LayerNorm
 * fused into in_proj and FF1, one persistent kernel for the whole batch,
 * x_proj fused into the scan, head.2 fused with the coder step.
 * boa_set_state_cache_budget sets the bytes of decode state kept in the
 * caches (< 0 restores the default, 160 MiB), which changes only the cache
 * policy of the state accesses, never the results. */
#define BOA_PLAN_FUSED_LN 1
#define BOA_PLAN_PERSISTENT 2
#define BOA_PLAN_FUSED_XPROJ 4
#define BOA_PLAN_FUSED_HEAD 8
int boa_decode_plan(const boa_ctx* ctx, int32_t lanes, int32_t* cached_layers, int32_t* flags);
int boa_set_state_cache_budget(boa_ctx* ctx, int64_t bytes);

/* Weights in the convert_boa_weights.py layout: "BOA\0" fp32, "BOA\1" fp16 or
 * headerless fp32.  Replaces BoaPredictorGPU::load_weights
 * (boa_gpu.hpp:990-1029); unlike the reference the file size is validated
 * against the configured dimensions. */
int boa_load_weights(boa_ctx* ctx, const char* path);
int boa_load_weights_mem(boa_ctx* ctx, const void* h_data, size_t n_bytes);
/* Expected weight-file size in bytes for a configuration. */
int64_t boa_weight_file_bytes(int32_t d_model, int32_t n_layers, int32_t d_state, int32_t fp16);

/* Device memory the context would use; replaces
 * BoaPredictorGPU::estimate_memory_static (boa_gpu.hpp:1103-1157). */
int64_t boa_estimate_memory(const boa_config* cfg, int64_t chunk_size, int32_t compress);

/* ---- model level (device pointers) ---------------------------------- */
/* Zero the recurrent conv and SSM state of the first `lanes` lanes;
 * replaces reset_cache (boa_gpu.hpp:249-252, 1159-1161). */
int boa_reset_state(boa_ctx* ctx, int32_t lanes);
/* Teacher-forced forward of T tokens per lane, state carried across calls:
 * d_tokens [lanes][T] -> d_logits [lanes][T][256] (head bias included).
 * Replaces BoaPredictorGPU::forward_chunk (boa_gpu.hpp:1081-1102). */
int boa_forward_chunk(boa_ctx* ctx, const uint8_t* d_tokens, int32_t lanes, int32_t T,
                      float* d_logits);
/* Allocation-free variant of boa_forward_chunk (no counterpart in the
 * reference).  For callers that cannot allocate device memory during the
 * call: code under HIP graph capture, tight serving loops, harnesses that
 * forbid hipMalloc.  Same inputs, outputs, state and results as
 * boa_forward_chunk, but the activations live in a fixed 64 MiB scratch
 * array per GPU (held until the process ends) instead of buffers the
 * context grows on demand; the call makes no hipMalloc, hipFree or other
 * allocating call.  Limit: lanes x T <= (64 MiB - 1792) / (4 (14 w +
 * ceil(d_model/16) + 2 d_state)) rows, w the built width d_model runs at
 * (4619 at d_model 256, d_state 16);
 * larger requests fail with BOA_E_ARG.  Every call on one GPU shares that
 * GPU's array: calls that overlap in time on one GPU (two host threads, or
 * two streams) race, so serialise them.  HIP-event profiling is off during
 * the call. */
int boa_forward_chunk_noalloc(boa_ctx* ctx, const uint8_t* d_tokens, int32_t lanes, int32_t T,
                              float* d_logits);
/* One decode step for every lane: d_tokens [lanes] -> d_logits [lanes][256];
 * add_bias = 0 leaves head.2's bias out as the decoder's call does.
 * Replaces BoaPredictorGPU::step_batch (boa_gpu.hpp:1034-1053). */
int boa_step_batch(boa_ctx* ctx, const uint8_t* d_tokens, int32_t lanes, float* d_logits,
                   int32_t add_bias);

/* ---- CDF and coder level (device pointers) ------------------------------ */
/* Integer CDFs of logits rows: d_qcdf [rows][257] with low_k in column k and
 * 2^24 in column 256; d_bias (may be NULL) is added first.  This is the CDF
 * stage of ker_rc_encode_chunk_parallel_warp / ker_rc_decode_fused_step_warp
 * (range_coder_kernels.cu:856-932, 504-570). */
int boa_cdf_from_logits(boa_ctx* ctx, const float* d_logits, const float* d_bias, int32_t rows,
                        uint32_t* d_qcdf);
/* Alternate CDF plug-in: the integer CDF the Python GPU codec builds from
 * probabilities (gpu_range_coder.py:57-79, build_cdf_fast), d_probs
 * [rows][K] -> d_qcdf [rows][K+1], K in [1, 1024].  The range coder of that
 * codec (gpu_range_coder.py:84-182) is the one behind boa_rc_encode_cdf /
 * boa_rc_decode_cdf (which take K = 256 rows), so probabilities computed
 * elsewhere can be coded into the Python codec's streams. */
int boa_cdf_from_probs(boa_ctx* ctx, const float* d_probs, int32_t rows, int32_t K,
                       uint32_t* d_qcdf);
/* Range-code explicit integer CDFs, one stream per lane: d_cdf
 * [lanes][n_sym][257], d_syms [lanes][n_sym] -> words at d_words + lane *
 * pitch_words, word counts in d_sizes.  Replaces gpu_rc_init +
 * the coder step + gpu_rc_finish_batch (gemm_gpu.hpp:194, 209). */
int boa_rc_encode_cdf(boa_ctx* ctx, const uint32_t* d_cdf, const uint8_t* d_syms, int32_t n_sym,
                      int32_t lanes, uint32_t* d_words, int64_t pitch_words, int32_t* d_sizes);
/* Inverse of boa_rc_encode_cdf; replaces gpu_rc_init_decoder and the
 * decoder step (gemm_gpu.hpp:220-223). */
int boa_rc_decode_cdf(boa_ctx* ctx, const uint32_t* d_cdf, int32_t n_sym, int32_t lanes,
                      const uint32_t* d_words, int64_t pitch_words, const int32_t* d_sizes,
                      uint8_t* d_syms);

/* ---- path level (device-resident data) ---------------------------------- */
/* Compress d_data[0, n) in chunks of chunk_size (at most max_chunks when
 * > 0).  Streams are written back to back into d_payload (capacity
 * payload_cap_words 32-bit words); per chunk the stream length in bytes and
 * the first byte are returned in host arrays of n_chunks entries.  Replaces
 * compress_v2's batch loop (boa.cpp:390-495) with on-device compaction. */
int boa_compress_device(boa_ctx* ctx, const uint8_t* d_data, int64_t n, int64_t chunk_size,
                        int32_t max_chunks, uint32_t* d_payload, int64_t payload_cap_words,
                        uint64_t* h_stream_bytes, uint8_t* h_first, int64_t* h_payload_words);
/* Number of chunks compress will produce (boa.cpp:295-298). */
int64_t boa_num_chunks(int64_t n, int64_t chunk_size, int32_t max_chunks);
/* Upper bound of the payload in words for boa_compress_device. */
int64_t boa_payload_bound_words(int64_t n, int64_t chunk_size, int32_t max_chunks);
/* Decompress streams stored back to back in d_payload (stream i starts at
 * 32-bit word h_offsets_words[i] and has h_stream_bytes[i] bytes) into
 * d_out[0, total).  Replaces decompress_v2's batch loop
 * (boa.cpp:672-774). */
int boa_decompress_device(boa_ctx* ctx, const uint32_t* d_payload, const uint64_t* h_offsets_words,
                          const uint64_t* h_stream_bytes, const uint8_t* h_first, int32_t n_chunks,
                          int64_t chunk_len, int64_t last_chunk_len, uint8_t* d_out);

/* ---- path level (host buffers / files, BOA2 container) ------------------ */
/* Compress a host buffer into a BOA2 container (malloc'd; free with
 * boa_free).  Replaces compress_v2 (boa.cpp:280-582); warm-start per
 * boa_set_warm_start. */
int boa_compress_buffer(boa_ctx* ctx, const uint8_t* h_in, int64_t n, int64_t chunk_size,
                        int32_t max_chunks, uint8_t** h_out, int64_t* out_len);
/* Decompress a BOA2 container; replaces decompress_v2 (boa.cpp:584-817). */
int boa_decompress_buffer(boa_ctx* ctx, const uint8_t* h_in, int64_t n, uint8_t** h_out,
                          int64_t* out_len);
/* Wall-clock phases of the last boa_compress_buffer / boa_decompress_buffer
 * (and so of the file calls): host-to-device copy, device work, device-to-
 * host copy, in seconds -- the H2D / Compute / D2H of boa.cpp's
 * --show-timings line (boa.cpp:504-507). */
int boa_last_timings(const boa_ctx* ctx, double* h2d_s, double* compute_s, double* d2h_s);
int boa_compress_file(boa_ctx* ctx, const char* in_path, const char* out_path, int64_t chunk_size,
                      int32_t max_chunks);
int boa_decompress_file(boa_ctx* ctx, const char* in_path, const char* out_path);
void boa_free(void* p);

/* ---- BOA2 container (host) ---------------------------------------------- */
/* CRC-32 (IEEE, reflected 0xEDB88320) as boa.cpp:85-107. */
uint32_t boa_crc32(const uint8_t* data, int64_t n);

/* ---- profiling: HIP events on the context stream ------------------------ */
#define BOA_K_GEMM 0       /* GEMMs on the 128x256 tile (compress bulk) */
#define BOA_K_SCAN 1
#define BOA_K_CONV 2
#define BOA_K_LN 3
#define BOA_K_CDF 4
#define BOA_K_CODER 5
#define BOA_K_DECODE 6     /* decode coder step (fp32: head.2 fused in) */
#define BOA_K_GEMM_SMALL 7 /* compress GEMMs on the smaller tile (x_proj) */
#define BOA_K_DEC_GEMM 8   /* decode-step GEMMs without a fused LayerNorm */
#define BOA_K_DEC_SCAN 9   /* decode-step scan (x_proj fused in where it runs so) */
#define BOA_K_HEAD_CDF 10  /* compress head.2 fused with the CDF (fp32) */
#define BOA_K_DEC_LNGEMM 11 /* decode-step LayerNorm + in_proj / FF1 GEMMs */
#define BOA_K_COUNT 12
/* When enabled, every kernel launch is bracketed by HIP events recorded on
 * the launch stream; boa_profile_read synchronises and returns, for a
 * kernel class, the summed kernel time (ms), the launch count and the
 * algorithmic work (FLOP for GEMM, bytes otherwise).  Reset clears totals. */
int boa_profile_enable(boa_ctx* ctx, int32_t on);
int boa_profile_reset(boa_ctx* ctx);
int boa_profile_read(boa_ctx* ctx, int32_t kernel_class, double* ms, int64_t* launches,
                     double* work);

#ifdef __cplusplus
}
#endif
#endif
