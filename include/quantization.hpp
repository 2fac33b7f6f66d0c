// Legacy quantisation dispatcher -- MI355X (gfx950) implementation.
//
// Drop-in replacement for the reference header
// legacy_modules/quantization/include/quantization/quantization.hpp:1-43 and
// the format structs of its impl headers (include/quantization/impl/*.hpp).
// The struct layouts below must stay identical to the reference (they are the
// serialised payload: quantization_get_packed_size bytes starting at the
// quantization_buffer_t), and the five functions keep C++ linkage with the
// reference's parameter types so that they mangle to the reference's symbol
// names.  include/bitsqz_llm_c.h declares extern "C" twins (bsq_legacy_*) and
// the device-pointer entry points.
//
// The codecs run on the GPU (csrc/legacy.hip): quantization_compress copies
// the input to the device, encodes it there and copies the payload back into
// one calloc'd block; quantization_decompress does the reverse.
#pragma once

#include <stdint.h>

#include "bitsqz_llm.hpp"  // quantization_method_t, BITSQZ_LLM_API

// --- format structs (reference include/quantization/impl/*.hpp) -----------

// q8_0_impl.hpp:10-16; block of 32, scale = absmax / 127.
typedef struct {
    unsigned long long num_elements;
    unsigned long long num_blocks;
    unsigned long long block_size;
    float *scales;
    int8_t *data;
} q8_0_array_t;

// q4_0_impl.hpp:11-17; block of 32, scale = absmax / 7, two codes per byte.
typedef struct {
    unsigned long long num_elements;
    unsigned long long num_blocks;
    unsigned long long block_size;
    float *scales;
    int8_t *data;
} q4_0_array_t;

// q2_k_impl.hpp:12-24; super-blocks of 16 blocks of 16 elements.
typedef struct {
    uint16_t super_scale;
    uint16_t super_min;
    uint8_t scales[16];
    uint8_t data[64];
} super_block_q2_k;

typedef struct {
    unsigned long long num_elements;
    unsigned long long num_elements_aligned;
    uint32_t num_super_blocks;
    super_block_q2_k *super_blocks;
} q2_k_array_t;

// bf16_impl.hpp:9-12, fp16_impl.hpp:9-12.
typedef struct {
    unsigned long long num_elements;
    uint16_t *data;
} bf16_array_t;

typedef struct {
    unsigned long long num_elements;
    uint16_t *data;
} fp16_array_t;

// fp8_impl.hpp:10-14, fp4_impl.hpp:10-14; one tensor-wide scale.
typedef struct {
    unsigned long long num_elements;
    float scale;
    uint8_t *data;
} fp8_array_t;

typedef struct {
    unsigned long long num_elements;
    float scale;
    uint8_t *data;
} fp4_array_t;

// mxfp8_impl.hpp:10-16, mxfp4_impl.hpp:10-16; power-of-two block scales.
typedef struct {
    unsigned long long num_elements;
    unsigned long long num_blocks;
    unsigned long long block_size;
    int8_t *scales;
    uint8_t *data;
} mxfp8_array_t;

typedef struct {
    unsigned long long num_elements;
    unsigned long long num_blocks;
    unsigned long long block_size;
    int8_t *scales;
    uint8_t *data;
} mxfp4_array_t;

// nvfp4_impl.hpp:11-18; tensor scale and E4M3 block scales over blocks of 16.
typedef struct {
    unsigned long long num_elements;
    unsigned long long num_blocks;
    unsigned long long block_size;
    float tensor_scale;
    uint8_t *block_scales;
    uint8_t *data;
} nvfp4_array_t;

// nf4_impl.hpp:10-16, nf4_dq_impl.hpp:17-24; blocks of 64.
typedef struct {
    unsigned long long num_elements;
    unsigned long long num_blocks;
    unsigned long long block_size;
    float *block_scales;
    uint8_t *data;
} nf4_array_t;

typedef struct {
    unsigned long long num_elements;
    unsigned long long num_blocks;
    unsigned long long block_size;
    float dq_scale;
    uint8_t *block_scales;
    uint8_t *data;
} nf4_dq_array_t;

// --- dispatcher (reference quantization.hpp:19-43) ------------------------

typedef struct {
    unsigned long long num_elements;
} quantization_shape_t;

typedef struct quantization_buffer {
    quantization_method_t method;
    quantization_shape_t shape;
    void *payload;
} quantization_buffer_t;

// Encodes `num_elements` host floats with `method` into a new buffer (one
// calloc'd block: this struct, then the format struct and its arrays); *out
// must be NULL.  Returns 0, or 1 on a bad argument, an unknown method or a
// failure (quantization.cpp:125-382).
BITSQZ_LLM_API int quantization_compress(const float *src, unsigned long long num_elements,
                                         quantization_method_t method, quantization_buffer_t **out);

// Decodes into `dst` (host, at least num_elements floats).  Returns 0, or 1
// on a bad argument or a buffer this build cannot decode (quantization.cpp:
// 384-460).
BITSQZ_LLM_API int quantization_decompress(const quantization_buffer_t *buf, float *dst,
                                           unsigned long long dst_num_elements);

// sizeof(quantization_buffer_t) + the payload size its header implies, or 0
// (quantization.cpp:462-467).
BITSQZ_LLM_API long long quantization_get_packed_size(const quantization_buffer_t *buf);

// A private copy of a serialised buffer with its pointers re-based, or NULL
// when the buffer is shorter than its header implies (quantization.cpp:469-484).
BITSQZ_LLM_API quantization_buffer_t *load_quantization_from_buffer(const void *buffer, long long buffer_size);

// Frees a buffer from quantization_compress / load_quantization_from_buffer.
BITSQZ_LLM_API void quantization_free(quantization_buffer_t *buf);
