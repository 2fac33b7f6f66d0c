// extern "C" entry points over the reference's legacy dispatcher
// (legacy_modules/quantization/src/quantization.cpp:125-489) and its eleven
// CPU codecs, compiled from the reference's own sources by oracle/Makefile
// into oracle/_ref/libref_legacy.so.  TEST INFRASTRUCTURE ONLY: it writes the
// golden vectors of tests/golden/legacy_golden.npz, pins oracle/legacy_oracle.c
// in the CPU tests where the reference tree exists, and is the "reference"
// CPU baseline of the legacy codecs; it is never shipped or measured as the
// product.
#include <quantization/datatype/bf16.hpp>
#include <quantization/datatype/fp16/fp16.hpp>
#include <quantization/quantization.hpp>

#include <omp.h>

#include <cstring>

extern "C" {

// OpenMP thread count of the reference's parallel loops; returns the count in
// effect.
__attribute__((visibility("default"))) int ref_legacy_set_threads(int n) {
    if (n > 0) omp_set_num_threads(n);
    return omp_get_max_threads();
}

// quantization_compress (quantization.cpp:125-382): copies the packed buffer
// (quantization_buffer_t followed by the payload, quantization_get_packed_size
// bytes) to `out` when it fits; returns that size, or -1 when compress fails.
__attribute__((visibility("default"))) long long ref_legacy_compress(int method, const float *x,
                                                                   unsigned long long n,
                                                                   unsigned char *out, long long cap) {
    quantization_buffer_t *buf = nullptr;
    if (quantization_compress(x, n, static_cast<quantization_method_t>(method), &buf) != 0 || !buf) return -1;
    const long long size = quantization_get_packed_size(buf);
    if (out && size <= cap) std::memcpy(out, buf, static_cast<size_t>(size));
    quantization_free(buf);
    return size;
}

// load_quantization_from_buffer + quantization_decompress
// (quantization.cpp:384-476); returns -1 when the load is refused, else the
// decompress status.
__attribute__((visibility("default"))) int ref_legacy_decompress(const unsigned char *packed, long long size,
                                                                 float *out, unsigned long long n) {
    quantization_buffer_t *buf = load_quantization_from_buffer(packed, size);
    if (!buf) return -1;
    const int rc = quantization_decompress(buf, out, n);
    quantization_free(buf);
    return rc;
}

// Timed legs of the CPU baseline: compress `reps` times (each result freed),
// then decompress the last result `reps` times into `out`.  Returns 0 on
// success.
__attribute__((visibility("default"))) int ref_legacy_roundtrip(int method, const float *x, unsigned long long n,
                                                                float *out, int reps, double *t_compress,
                                                                double *t_decompress) {
    quantization_buffer_t *buf = nullptr;
    const double t0 = omp_get_wtime();
    for (int r = 0; r < reps; ++r) {
        if (buf) quantization_free(buf);
        buf = nullptr;
        if (quantization_compress(x, n, static_cast<quantization_method_t>(method), &buf) != 0 || !buf) return 1;
    }
    const double t1 = omp_get_wtime();
    for (int r = 0; r < reps; ++r)
        if (quantization_decompress(buf, out, n) != 0) return 1;
    const double t2 = omp_get_wtime();
    quantization_free(buf);
    *t_compress = (t1 - t0) / reps;
    *t_decompress = (t2 - t1) / reps;
    return 0;
}

// The reference's scalar conversions (datatype/fp16/fp16.hpp,
// datatype/bf16.hpp) over every float pattern in [lo, hi): kind 0 FP16,
// kind 1 BF16; sum of (result + 1) * (pattern mod 65521), mod 2^64.
__attribute__((visibility("default"))) unsigned long long ref_legacy_sweep(int kind, unsigned long long lo,
                                                                          unsigned long long hi) {
    unsigned long long acc = 0;
    for (unsigned long long p = lo; p < hi; ++p) {
        const uint32_t u = static_cast<uint32_t>(p);
        float f;
        std::memcpy(&f, &u, 4);
        const unsigned long long r = kind == 0 ? fp16_ieee_from_fp32_value(f) : bf16_from_fp32_value(f);
        acc += (r + 1) * (p % 65521u);
    }
    return acc;
}

// FP16 -> FP32 of one pattern (fp16.hpp:73-95).
__attribute__((visibility("default"))) float ref_legacy_fp16_to_f32(unsigned short h) {
    return fp16_ieee_to_fp32_value(h);
}

}  // extern "C"
