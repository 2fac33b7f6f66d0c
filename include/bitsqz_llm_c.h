/*
 * bitsqz_llm C-ABI boundary -- MI355X (gfx950).
 *
 * Plain extern "C" entry points (plain pointers and sizes, no HIP or torch
 * types) for FFI callers: Python ctypes, cgo, JNI, N-API.  Device pointers are
 * passed as ordinary pointers; `stream` is a hipStream_t passed as void*
 * (NULL = the HIP null stream).  Every int-returning function returns 0 on
 * success and 1 on failure (the reference convention, src/bitsqz_llm.cu);
 * bsq_last_error() returns the message of the most recent failure on the
 * calling thread.
 *
 * Three groups:
 *   1. bsq_*          -- extern "C" twins of the nine C++-linkage ABI
 *                        functions in bitsqz_llm.hpp (same semantics).
 *   2. bsq_device_*   -- the same compress / decompress pipeline with the
 *                        packed sections kept in device memory (no host
 *                        round trip, no host synchronisation); used to measure
 *                        the device-resident path and by the host ABI itself.
 *   3. bsq_topk_*, bsq_quant_*, bsq_svd_*, bsq_reconstruct_* -- the four
 *                        module operators the pipeline is built from, each
 *                        mirroring a reference module entry point.
 */
#ifndef BITSQZ_LLM_C_H
#define BITSQZ_LLM_C_H

#include <stdint.h>

#include "bitsqz_llm.hpp"

#ifdef __cplusplus
extern "C" {
#endif

#define BSQ_API __attribute__((visibility("default")))

/* ---------------------------------------------------------------------------
 * 0. Diagnostics
 * ------------------------------------------------------------------------- */

/* Message of the last failure on this thread ("" if none).  No reference
 * counterpart: the reference discards exception messages at the boundary
 * (src/bitsqz_llm.cu:878-881). */
BSQ_API const char *bsq_last_error(void);

/* Library version string. */
BSQ_API const char *bsq_version(void);

/* ---------------------------------------------------------------------------
 * 1. extern "C" twins of the C++ ABI (include/bitsqz_llm.hpp)
 * ------------------------------------------------------------------------- */

/* replaces bitsqz_llm_compress_initialize, reference bitsqz_llm.hpp:95-105 */
BSQ_API int bsq_compress_initialize(uint16_t num_rows, uint16_t num_columns,
                                    float outlier_topk_ratio, float error_correction_topk_ratio,
                                    int svd_ranks, int svd_niters,
                                    int svd_uv_format, int svd_s_format,
                                    int quantization_only_format, int input_location);
/* replaces bitsqz_llm_compress_release, reference bitsqz_llm.hpp:107 */
BSQ_API void bsq_compress_release(void);
/* replaces bitsqz_llm_decompress_initialize, reference bitsqz_llm.hpp:109-117 */
BSQ_API int bsq_decompress_initialize(uint16_t num_rows, uint16_t num_columns,
                                      float outlier_topk_ratio, float error_correction_topk_ratio,
                                      int svd_ranks, int svd_uv_format, int svd_s_format,
                                      int quantization_only_format);
/* replaces bitsqz_llm_decompress_release, reference bitsqz_llm.hpp:119 */
BSQ_API void bsq_decompress_release(void);
/* replaces bitsqz_llm_compress, reference bitsqz_llm.hpp:121-124 */
BSQ_API int bsq_compress(const float *row_major_matrix_float_data, bitsqz_llm_array_t **out,
                         bitsqz_llm_compress_profile_t *profile);
/* replaces bitsqz_llm_decompress, reference bitsqz_llm.hpp:132-135 */
BSQ_API int bsq_decompress(const bitsqz_llm_array_t *compressed, float *d_dst,
                           uint32_t dst_num_elements);
/* replaces bitsqz_llm_get_packed_size, reference bitsqz_llm.hpp:137 */
BSQ_API uint64_t bsq_get_packed_size(const bitsqz_llm_array_t *compressed);
/* replaces load_bitsqz_llm_from_buffer, reference bitsqz_llm.hpp:139 */
BSQ_API bitsqz_llm_array_t *bsq_load_from_buffer(const void *buffer, uint64_t buffer_size);
/* replaces bitsqz_llm_free, reference bitsqz_llm.hpp:141 */
BSQ_API void bsq_free(bitsqz_llm_array_t *compressed);

/* Test hook: replace the Gaussian sketch of the compress runtime's SVD by a
 * caller-supplied device matrix (N_work x rank, row-major, N_work =
 * min(rows, cols)); NULL restores the built-in generator.  The reference
 * draws the sketch from cuRAND inside a CUDA graph
 * (modules/svd_lowrank_cuda/src/svd_lowrank_cuda.cu:289-291, 552-556), which
 * no other implementation can reproduce, so parity of the SVD path is defined
 * with an injected sketch.  The pointer must stay valid while it is set. */
BSQ_API int bsq_compress_set_sketch(const float *d_sketch);

/* ---------------------------------------------------------------------------
 * 2. Device-resident pipeline
 * ------------------------------------------------------------------------- */

/* A packed object whose sections live in device memory.  `header` carries the
 * header fields the host object would have (section offsets/sizes are
 * payload-relative, `payload` is NULL) with the flags the host can decide
 * (SVD, outlier).  Whether the error-correction section is present is decided
 * on the device: the word *d_flags (device memory) has bit 2 set when it is,
 * and header.section_error_topk describes it for that case.  The component
 * pointers are device pointers owned by the compress runtime; they stay valid
 * until the next compress call or release.  For quantised sections d_dense is
 * NULL and the scales / codes pointers are set; for FP32 sections d_dense is
 * set. */
typedef struct {
    bitsqz_llm_array_t header;
    const uint32_t *d_flags;
    /* quantised / dense sections: U, S, V, direct (index 0..3) */
    const float *d_dense[4];        /* FP32 storage (section stored dense) */
    const float *d_scales_f32[4];   /* NF4 block scales                      */
    const uint8_t *d_scales_u8[4];  /* NF4_DQ E4M3 block scale codes         */
    const float *d_dq_scale[4];     /* NF4_DQ global scale (1 float)         */
    const uint8_t *d_codes[4];      /* packed nibbles                        */
    uint64_t count[4];              /* element count of each section         */
    /* top-k sections: outlier (0), error (1) */
    const uint16_t *d_topk_idx[2];
    const float *d_topk_val[2];
    uint16_t topk_k[2];
} bsq_device_packed_t;

/* Run the whole compress pipeline of the initialised compress runtime on
 * `d_input` (device memory, row-major rows x cols), enqueued on the runtime's
 * stream; returns without a host synchronisation. */
BSQ_API int bsq_device_compress(const float *d_input, bsq_device_packed_t *out);

/* Decode a device-resident packed object into `d_dst` with the initialised
 * decompress runtime (same configuration checks as bsq_decompress), enqueued
 * on the compress runtime's stream when one exists; no host synchronisation. */
BSQ_API int bsq_device_decompress(const bsq_device_packed_t *packed, float *d_dst,
                                  uint32_t dst_num_elements);

/* Wait for all work the runtimes enqueued. */
BSQ_API int bsq_device_synchronize(void);

/* The stream the runtimes enqueue on (a hipStream_t). */
BSQ_API void *bsq_runtime_stream(void);

/* Lanes (no counterpart in the reference, whose runtimes are process-global
 * singletons, src/bitsqz_llm.cu:33-138): `lanes` (1..8) independent pairs of
 * compress + decompress runtimes with the given configuration (DEVICE input;
 * the decompress runtime takes the effective rank), each on its own stream.
 * bsq_lanes_roundtrip enqueues one device-resident compress of d_input and
 * the decompress of its result into d_dst (rows x cols floats) on the lane's
 * stream, exactly as bsq_device_compress + bsq_device_decompress do, and
 * returns without a host synchronisation.  Lanes share no buffers, so round
 * trips on different lanes run concurrently; a lane's packed object lives
 * until its next round trip.  For callers with several matrices in flight
 * (e.g. the activations of several layers). */
BSQ_API int bsq_lanes_initialize(int lanes, uint16_t rows, uint16_t cols, float outlier_topk_ratio,
                                 float error_correction_topk_ratio, int svd_ranks, int svd_niters,
                                 int svd_uv_format, int svd_s_format, int quantization_only_format);
BSQ_API int bsq_lanes_roundtrip(int lane, const float *d_input, float *d_dst);
BSQ_API void *bsq_lanes_stream(int lane);
BSQ_API int bsq_lanes_synchronize(void);
BSQ_API void bsq_lanes_release(void);

/* ---------------------------------------------------------------------------
 * 3. Module operators
 * ------------------------------------------------------------------------- */

/* k = roundf(cols * ratio), clamped to [1, cols] when ratio > 0.
 * replaces topk_compute_num_topk_columns, reference
 * modules/topk_cuda/src/topk_cuda.cu:53-69 (which throws on a bad ratio;
 * here: returns 1). */
BSQ_API int bsq_topk_num_columns(uint16_t num_columns, float ratio, uint16_t *out_k);

/* Per-row top-k of |x| (NaN ranks lowest), ordered by |x| descending with
 * ties to the lower column; writes indices[r*k + j] and the signed values.
 * If d_residual is not NULL it receives the input with the selected entries
 * zeroed (it may alias d_input: in-place separation).
 * replaces topk_extraction / topk_separation, reference
 * modules/topk_cuda/src/topk_cuda.cu:186-201. */
BSQ_API int bsq_topk_select(const float *d_input, uint16_t rows, uint16_t cols, uint16_t k,
                            uint16_t *d_indices, float *d_values, float *d_residual,
                            void *stream);

/* dense[r, idx] += value for every entry (topk_apply, reference
 * modules/topk_cuda/src/topk_cuda.cu:221-233) or, with accumulate == 0,
 * dense = 0 then dense[r, idx] = value (topk_decompress, :203-219). */
BSQ_API int bsq_topk_scatter(const uint16_t *d_indices, const float *d_values, uint16_t rows,
                             uint16_t cols, uint16_t k, float *d_dense, int accumulate,
                             void *stream);

/* NF4 (method 11) or NF4_DQ (method 10) block-64 quantisation of `count`
 * floats.  NF4 writes d_scales_f32[ceil(count/64)]; NF4_DQ writes
 * d_scales_u8[ceil(count/64)] and *d_dq_scale.  Codes: ceil(count/2) bytes.
 * replaces quantization_cuda_compress, reference
 * modules/quantization_cuda/src/quantization_cuda.cu:564-624. */
BSQ_API int bsq_quant_compress(const float *d_input, uint64_t count, int method,
                               float *d_scales_f32, uint8_t *d_scales_u8, float *d_dq_scale,
                               uint8_t *d_codes, void *stream);

/* replaces quantization_cuda_decompress, reference
 * modules/quantization_cuda/src/quantization_cuda.cu:626-663. */
BSQ_API int bsq_quant_decompress(uint64_t count, int method, const float *d_scales_f32,
                                 const uint8_t *d_scales_u8, const float *d_dq_scale,
                                 const uint8_t *d_codes, float *d_output, void *stream);

/* Test hooks for the scalar codec primitives (reference
 * quantization_cuda.cu:43-128): NF4 nearest-code of each value, E4M3 encode of
 * each value, E4M3 decode of each code. */
BSQ_API int bsq_quant_nf4_codes(const float *d_values, uint64_t n, uint8_t *d_codes, void *stream);
BSQ_API int bsq_quant_e4m3_encode(const float *d_values, uint64_t n, uint8_t *d_codes, void *stream);
BSQ_API int bsq_quant_e4m3_decode(const uint8_t *d_codes, uint64_t n, float *d_values, void *stream);

/* NF4 code of every float bit pattern in [lo, hi) (hi <= 2^32): 16-bin
 * histogram and sum over patterns of code * (pattern mod 65521), written to
 * device memory; pins the device code function against a CPU sweep. */
BSQ_API int bsq_quant_nf4_code_sweep(uint64_t lo, uint64_t hi, unsigned long long *d_hist16,
                                     unsigned long long *d_checksum, void *stream);
/* The 15 exact decision thresholds the device NF4 code function uses for
 * |v| < 2 (code = number of thresholds <= v). */
BSQ_API void bsq_nf4_thresholds(float out[15]);

/* Randomised rank-q SVD of a row-major m x n matrix with `niter` power
 * iterations and no oversampling: U (m x q), S (q), V (n x q), row-major,
 * q = max(1, min(q, m, n)).  d_sketch (min(m,n) x q, row-major) may be NULL
 * to draw the sketch from the built-in generator with `seed`.
 * replaces svd_lowrank_cuda, reference
 * modules/svd_lowrank_cuda/src/svd_lowrank_cuda.cu:541-581. */
BSQ_API int bsq_svd_lowrank(const float *d_A, int m, int n, int q, int niter,
                            const float *d_sketch, uint64_t seed, float *d_U, float *d_S,
                            float *d_V, void *stream);

/* bsq_svd_lowrank without any device allocation.  No counterpart in the
 * reference: for callers that cannot allocate device memory (code under HIP
 * graph capture, allocation-free serving loops).  Same arguments and results
 * as bsq_svd_lowrank (the same kernels on the same plan layout), but the
 * plan's buffers are carved from the library's fixed 256 MiB device array
 * (one copy per GPU, held until the process ends), so shapes whose plan needs
 * more return 1 with the byte counts in bsq_last_error().  Asynchronous on
 * `stream` (no synchronisation); calls that overlap on one GPU share that
 * array and race. */
BSQ_API int bsq_svd_lowrank_noalloc(const float *d_A, int m, int n, int q, int niter,
                                    const float *d_sketch, uint64_t seed, float *d_U,
                                    float *d_S, float *d_V, void *stream);

/* out (m x n, row-major) = U (m x k) * diag(S) * V (n x k)^T.
 * replaces reconstruct_lowrank_cuda, reference
 * modules/reconstruct_lowrank_cuda/src/reconstruct_lowrank_cuda.cu:21-62,153-171. */
BSQ_API int bsq_reconstruct_lowrank(const float *d_U, const float *d_S, const float *d_V, int m,
                                    int n, int k, float *d_out, void *stream);

/* Fill `n` floats with N(0,1) draws of the built-in sketch generator
 * (counter-based Philox4x32-10 + Box-Muller; deterministic in (seed, index)). */
BSQ_API int bsq_gaussian_fill(float *d_out, uint64_t n, uint64_t seed, void *stream);

/* ---------------------------------------------------------------------------
 * 4. Device memory helpers for FFI callers without a GPU framework (no
 *    reference counterpart; thin wrappers over hipMalloc / hipMemcpy).
 * ------------------------------------------------------------------------- */
BSQ_API int bsq_device_count(int *count);
BSQ_API int bsq_device_malloc(void **ptr, uint64_t bytes);
BSQ_API int bsq_device_free(void *ptr);
BSQ_API int bsq_memcpy_h2d(void *dst, const void *src, uint64_t bytes);
BSQ_API int bsq_memcpy_d2h(void *dst, const void *src, uint64_t bytes);
BSQ_API int bsq_memcpy_d2d(void *dst, const void *src, uint64_t bytes);
BSQ_API int bsq_device_memset(void *dst, int value, uint64_t bytes);
/* Pinned (page-locked) host memory, hipHostMalloc / hipHostFree, and an
 * asynchronous host-to-device copy on a caller-chosen stream (null: the
 * default stream). */
BSQ_API int bsq_host_malloc(void **ptr, uint64_t bytes);
BSQ_API int bsq_host_free(void *ptr);
BSQ_API int bsq_memcpy_h2d_async(void *dst, const void *src, uint64_t bytes, void *stream);
BSQ_API int bsq_stream_synchronize(void *stream);
/* HIP events on a caller-chosen stream (timing without a GPU framework). */
BSQ_API int bsq_event_create(void **event);
BSQ_API int bsq_event_destroy(void *event);
BSQ_API int bsq_event_record(void *event, void *stream);
BSQ_API int bsq_event_elapsed_ms(void *start, void *stop, float *ms);

/* Instrumentation (no counterpart in the reference): while started, the
 * launches of six classes inside the compress / decompress pipelines are
 * bracketed by HIP events on their own stream.  _stop waits for those events
 * and returns the summed time and launch count of the low-rank reconstruction
 * GEMMs; _read then returns any class: 0 = reconstruction GEMM, 1 = the range
 * finder's products with the big matrix (split-K / stream-K reductions
 * included), 2 = outlier separation top-k, 3 = error-correction top-k,
 * 4 = direct-section encode (with the NF4_DQ global-scale reduce),
 * 5 = direct-section decode (with the fused top-k scatter). */
BSQ_API int bsq_kernel_timer_start(void);
BSQ_API int bsq_kernel_timer_read(int timer_class, double *total_ms, int *launches);
/* Plain device copy kernel (16 bytes per lane), the known-size reference for
 * calibrating HBM byte counters.  bytes and both pointers 16-byte aligned. */
BSQ_API int bsq_copy_kernel(const void *d_src, void *d_dst, uint64_t bytes, void *stream);
BSQ_API int bsq_kernel_timer_stop(double *total_ms, int *launches);

/* ---------------------------------------------------------------------------
 * 5. Legacy quantisation formats (include/quantization.hpp): the reference's
 *    CPU codec dispatcher, here encoding and decoding on the GPU.
 * ------------------------------------------------------------------------- */
/* extern "C" twins of the five C++-linkage functions of include/quantization.hpp;
 * replace quantization_compress / quantization_decompress /
 * quantization_get_packed_size / load_quantization_from_buffer /
 * quantization_free, reference
 * legacy_modules/quantization/src/quantization.cpp:125-489.  `method` is a
 * quantization_method_t value; buffers are quantization_buffer_t *. */
BSQ_API int bsq_legacy_compress(int method, const float *src, uint64_t n, void **out);
BSQ_API int bsq_legacy_decompress(const void *buf, float *dst, uint64_t n);
BSQ_API long long bsq_legacy_packed_size(const void *buf);
BSQ_API void *bsq_legacy_load(const void *buffer, long long size);
BSQ_API void bsq_legacy_free(void *buf);

/* Bytes of the payload (format struct + arrays) of n elements, or -1.  The
 * reference's get_*_array_size (e.g. q8_0_impl.cpp:3-6) on the struct that
 * its compress writes. */
BSQ_API long long bsq_legacy_payload_bytes(int method, uint64_t n);

/* Device-resident codec (no reference counterpart: the reference codecs take
 * host arrays).  Encode writes the payload image of n device floats to
 * d_payload (16-byte aligned, bsq_legacy_payload_bytes bytes): the format
 * struct with its counts and scale, then its arrays, byte-identical to the
 * reference's payload except the struct's pointer fields, which are left
 * unspecified (FP8, FP4, NVFP4 and NF4_DQ use one as reduction scratch).
 * Decode reads such an image of n elements.  Asynchronous on `stream`. */
BSQ_API int bsq_legacy_encode_device(int method, const float *d_src, uint64_t n, void *d_payload,
                                     void *stream);
BSQ_API int bsq_legacy_decode_device(int method, const void *d_payload, uint64_t n, float *d_dst,
                                     void *stream);

/* Test hook: adds to *d_checksum the sum over float patterns p in [lo, hi)
 * (hi <= 2^32) of (r(p) + 1) * (p mod 65521), where r is the device FP16
 * conversion (kind 0), BF16 conversion (1) or MX block exponent as a byte
 * (2: max norm 448, 3: max norm 6). */
BSQ_API int bsq_legacy_sweep(int kind, uint64_t lo, uint64_t hi, unsigned long long *d_checksum,
                             void *stream);

#ifdef __cplusplus
}
#endif

#endif /* BITSQZ_LLM_C_H */
