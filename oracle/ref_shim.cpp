// extern "C" entry points over the reference's legacy NF4 / NF4_DQ CPU codec
// (legacy_modules/quantization/src/impl/nf4_impl.cpp, nf4_dq_impl.cpp),
// compiled from the reference's own sources by oracle/Makefile into
// oracle/_ref/libref_nf4.so.  TEST INFRASTRUCTURE ONLY: used to write the
// golden vectors and as the "reference" CPU baseline; never shipped or
// measured as the product.
#include <quantization/impl/nf4_dq_impl.hpp>
#include <quantization/impl/nf4_impl.hpp>

#include <omp.h>

#include <cstring>

extern "C" {

// Sets the OpenMP thread count the reference codec's parallel loops use
// (nf4_impl.cpp:104, nf4_dq_impl.cpp:174,197,255) and returns the count in
// effect, so a timing reports the threads that actually ran.
__attribute__((visibility("default"))) int ref_set_threads(int n) {
    if (n > 0) omp_set_num_threads(n);
    return omp_get_max_threads();
}

// Runs nf4_compress (nf4_impl.cpp:92-135) and copies the block scales and
// codes out of the reference's own allocation.
__attribute__((visibility("default"))) int ref_nf4_compress(const float *x, unsigned long long n,
                                                            float *scales, unsigned char *codes) {
    nf4_array_t *arr = nullptr;
    if (nf4_compress(x, n, &arr) != 0 || arr == nullptr) return 1;
    std::memcpy(scales, arr->block_scales, arr->num_blocks * sizeof(float));
    std::memcpy(codes, arr->data, (n + 1) / 2);
    free_nf4_array(arr);
    return 0;
}

// Builds an nf4_array_t from caller buffers and runs nf4_decompress
// (nf4_impl.cpp:137-164).
__attribute__((visibility("default"))) int ref_nf4_decompress(const float *scales,
                                                              const unsigned char *codes,
                                                              unsigned long long n, float *out) {
    nf4_array_t *arr = allocate_nf4_array(n, DEFAULT_NF4_BLOCK_SIZE);
    if (!arr) return 1;
    std::memcpy(arr->block_scales, scales, arr->num_blocks * sizeof(float));
    std::memcpy(arr->data, codes, (n + 1) / 2);
    const int rc = nf4_decompress(arr, out);
    free_nf4_array(arr);
    return rc;
}

// nf4_dq_compress (nf4_dq_impl.cpp:227-242).
__attribute__((visibility("default"))) int ref_nf4dq_compress(const float *x, unsigned long long n,
                                                              float *dq, unsigned char *scale_codes,
                                                              unsigned char *codes) {
    nf4_dq_array_t *arr = nullptr;
    if (nf4_dq_compress(x, n, &arr) != 0 || arr == nullptr) return 1;
    *dq = arr->dq_scale;
    std::memcpy(scale_codes, arr->block_scales, arr->num_blocks);
    std::memcpy(codes, arr->data, (n + 1) / 2);
    free_nf4_dq_array(arr);
    return 0;
}

// nf4_dq_decompress (nf4_dq_impl.cpp:244-275).
__attribute__((visibility("default"))) int ref_nf4dq_decompress(float dq,
                                                                const unsigned char *scale_codes,
                                                                const unsigned char *codes,
                                                                unsigned long long n, float *out) {
    nf4_dq_array_t *arr = allocate_nf4_dq_array(n, DEFAULT_NF4_DQ_BLOCK_SIZE);
    if (!arr) return 1;
    arr->dq_scale = dq;
    std::memcpy(arr->block_scales, scale_codes, arr->num_blocks);
    std::memcpy(arr->data, codes, (n + 1) / 2);
    const int rc = nf4_dq_decompress(arr, out);
    free_nf4_dq_array(arr);
    return rc;
}
}
