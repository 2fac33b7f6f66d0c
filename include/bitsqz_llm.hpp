// bitsqz_llm public ABI -- MI355X (gfx950) implementation.
//
// Drop-in replacement for the reference header include/bitsqz_llm.hpp:1-141.
// Every type, enumerator value, field order and function signature below must
// stay identical to the reference so that (a) the nine C++-linkage symbols
// mangle to the same names and (b) sizeof(bitsqz_llm_array_t) == 200 with the
// section descriptors at byte offsets 48/72/96/120/144/168 and the payload
// self-pointer at 192.  The functions keep C++ linkage (no extern "C") for the
// same reason; include/bitsqz_llm_c.h exposes extern "C" equivalents for FFI
// callers (ctypes, cgo, JNI).
#pragma once

#include <stdint.h>

#if defined(_WIN32)
#if defined(BITSQZ_LLM_EXPORTS)
#define BITSQZ_LLM_API __declspec(dllexport)
#else
#define BITSQZ_LLM_API __declspec(dllimport)
#endif
#else
#define BITSQZ_LLM_API __attribute__((visibility("default")))
#endif

#ifndef BITSQZ_LLM_QUANTIZATION_METHOD_T_DEFINED
#define BITSQZ_LLM_QUANTIZATION_METHOD_T_DEFINED
// Quantisation formats (reference bitsqz_llm.hpp:17-33).  Only NONE, NF4 and
// NF4_DQ are accepted by the runtime; the other values exist so that the enum
// (and therefore the mangled symbol names) match.
typedef enum {
    quantization_NONE = -1,
    quantization_INVALID = quantization_NONE,
    Q8_0 = 0,
    Q4_0 = 1,
    Q2_K = 2,
    BF16 = 3,
    FP16 = 4,
    FP8 = 5,
    FP4 = 6,
    MXFP8 = 7,
    MXFP4 = 8,
    NVFP4 = 9,
    NF4_DQ = 10,
    NF4 = 11,
    Q2_K_FAST = 12,
} quantization_method_t;
#endif

// Section storage kinds (reference bitsqz_llm.hpp:36-41).
typedef enum {
    BITSQZ_SECTION_NONE = 0,
    BITSQZ_SECTION_FP32 = 1,
    BITSQZ_SECTION_QUANT = 2,
    BITSQZ_SECTION_TOPK = 3,
} bitsqz_section_storage_t;

// Where the compress input lives (reference bitsqz_llm.hpp:43-46).
typedef enum {
    BITSQZ_LLM_INPUT_HOST = 0,
    BITSQZ_LLM_INPUT_DEVICE = 1,
} bitsqz_llm_input_location_t;

// 24-byte section descriptor; offset is relative to the payload start
// (reference bitsqz_llm.hpp:48-53).
typedef struct {
    uint64_t offset;
    uint64_t size;
    uint8_t storage;
    uint8_t reserved[7];
} bitsqz_section_t;

// 200-byte packed-object header; the payload follows it in the same
// allocation (reference bitsqz_llm.hpp:55-83).
typedef struct bitsqz_llm_array {
    uint16_t num_rows;
    uint16_t num_columns;
    uint32_t num_elements;

    float outlier_topk_ratio;
    float error_correction_topk_ratio;

    int16_t svd_ranks;
    int16_t svd_niters;
    int16_t effective_rank;
    int16_t reserved0;

    quantization_method_t svd_uv_format;
    quantization_method_t svd_s_format;
    quantization_method_t quantization_only_format;
    int32_t reserved1;

    uint32_t flags;

    bitsqz_section_t section_u;
    bitsqz_section_t section_s;
    bitsqz_section_t section_v;
    bitsqz_section_t section_direct;
    bitsqz_section_t section_outlier_topk;
    bitsqz_section_t section_error_topk;

    void *payload;
} bitsqz_llm_array_t;

// Per-stage compress latencies in milliseconds (reference bitsqz_llm.hpp:85-93).
// The misspelled field name is part of the ABI and is kept verbatim.
typedef struct {
    double topk_separation_latency_ms;
    double svd_lowrank_cuda_latency_ms;
    double quantization_compress_latency_ms;
    double reconsturct_quantization_decompress_latency_ms;
    double reconstruct_svd_latency_ms;
    double error_extraction_latency_ms;
    double other_latency_ms;
} bitsqz_llm_compress_profile_t;

// reference bitsqz_llm.hpp:95-105
BITSQZ_LLM_API int bitsqz_llm_compress_initialize(
    uint16_t num_rows,
    uint16_t num_columns,
    float outlier_topk_ratio,
    float error_correction_topk_ratio,
    int svd_ranks,
    int svd_niters,
    quantization_method_t svd_uv_format,
    quantization_method_t svd_s_format,
    quantization_method_t quantization_only_format,
    bitsqz_llm_input_location_t input_location);

// reference bitsqz_llm.hpp:107
BITSQZ_LLM_API void bitsqz_llm_compress_release();

// reference bitsqz_llm.hpp:109-117
BITSQZ_LLM_API int bitsqz_llm_decompress_initialize(
    uint16_t num_rows,
    uint16_t num_columns,
    float outlier_topk_ratio,
    float error_correction_topk_ratio,
    int svd_ranks,
    quantization_method_t svd_uv_format,
    quantization_method_t svd_s_format,
    quantization_method_t quantization_only_format);

// reference bitsqz_llm.hpp:119
BITSQZ_LLM_API void bitsqz_llm_decompress_release();

// reference bitsqz_llm.hpp:121-124
BITSQZ_LLM_API int bitsqz_llm_compress(
    const float *row_major_matrix_float_data,
    bitsqz_llm_array_t **out,
    bitsqz_llm_compress_profile_t *profile);

// reference bitsqz_llm.hpp:126-130 (header-inline convenience overload)
inline int bitsqz_llm_compress(
    const float *row_major_matrix_float_data,
    bitsqz_llm_array_t **out) {
    return bitsqz_llm_compress(row_major_matrix_float_data, out, nullptr);
}

// reference bitsqz_llm.hpp:132-135
BITSQZ_LLM_API int bitsqz_llm_decompress(
    const bitsqz_llm_array_t *compressed,
    float *d_dst,
    uint32_t dst_num_elements);

// reference bitsqz_llm.hpp:137
BITSQZ_LLM_API uint64_t bitsqz_llm_get_packed_size(const bitsqz_llm_array_t *compressed);

// reference bitsqz_llm.hpp:139
BITSQZ_LLM_API bitsqz_llm_array_t *load_bitsqz_llm_from_buffer(const void *buffer, uint64_t buffer_size);

// reference bitsqz_llm.hpp:141
BITSQZ_LLM_API void bitsqz_llm_free(bitsqz_llm_array_t *compressed);
