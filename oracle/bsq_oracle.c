/*
 * bitsqz_llm CPU oracle -- TEST INFRASTRUCTURE ONLY.
 *
 * A plain-C restatement of the reference's integer/byte arithmetic on the
 * compress/decompress hot path.  It is the checker for the HIP library: only
 * tests/, __graft_entry__.smoke() and bench.py's cpu_baseline leg may load it,
 * and never as the thing that is measured or shipped.
 *
 * Each function cites the reference file:line it follows.  The NF4 / NF4_DQ /
 * E4M3 codecs follow the legacy CPU codec, which the reference's own test
 * (tests/quantization_cuda/test_nf4_cuda.cu:109-114) requires to equal the
 * CUDA codec bit for bit.  Pinning: tests/test_oracle.py checks every function
 * here against the golden vectors in tests/golden/ (written by the reference's
 * legacy codec compiled from its own sources, oracle/Makefile) and against
 * closed forms / brute force.
 *
 * Build: oracle/Makefile -> oracle/liboracle.so (g++ is not needed; plain C99
 * + OpenMP).  Compiled with -ffp-contract=off so no multiply-subtract is fused.
 */
#include <math.h>
#include <stdint.h>
#include <stdlib.h>
#include <string.h>

#define ORACLE_API __attribute__((visibility("default")))

/* NF4 code book (legacy_modules/quantization/src/impl/nf4_impl.cpp:3-20). */
static const float kLevels[16] = {
    -1.0f,
    -0.6961928009986877f,
    -0.5250730514526367f,
    -0.39491748809814453f,
    -0.28444138169288635f,
    -0.18477343022823334f,
    -0.09105003625154495f,
    0.0f,
    0.07958029955625534f,
    0.16093020141124725f,
    0.24611230194568634f,
    0.33791524171829224f,
    0.44070982933044434f,
    0.5626170039176941f,
    0.7229568362236023f,
    1.0f,
};

ORACLE_API const float *oracle_nf4_levels(void) { return kLevels; }

/* Nearest code with first-minimum tie break: linear scan with strict '<'
 * (nf4_impl.cpp:73-86; identical in nf4_dq_impl.cpp:131-144 and
 * quantization_cuda.cu:43-58).  Non-finite input maps to 0.0. */
ORACLE_API uint8_t oracle_nf4_code(float x) {
    if (!isfinite(x)) x = 0.0f;
    int best = 0;
    float best_err = fabsf(x - kLevels[0]);
    for (int i = 1; i < 16; ++i) {
        const float err = fabsf(x - kLevels[i]);
        if (err < best_err) {
            best_err = err;
            best = i;
        }
    }
    return (uint8_t)best;
}

/* Block absmax over a (possibly partial) block, non-finite treated as 0;
 * an all-zero block gets scale 1.0 (nf4_impl.cpp:110-117). */
static float block_absmax(const float *x, uint64_t start, uint64_t remain) {
    float m = 0.0f;
    for (uint64_t i = 0; i < remain; ++i) {
        float v = x[start + i];
        if (!isfinite(v)) v = 0.0f;
        const float a = fabsf(v);
        if (a > m) m = a;
    }
    return m;
}

static void encode_block(const float *x, uint64_t start, uint64_t remain, float inv,
                         uint8_t *codes) {
    /* nf4_impl.cpp:121-130: multiply by the reciprocal, nearest code, even
     * element -> high nibble, odd element -> low nibble. */
    for (uint64_t i = 0; i < remain; ++i) {
        const float v = x[start + i] * inv;
        const uint8_t c = oracle_nf4_code(v) & 0xF;
        const uint64_t e = start + i;
        if ((e & 1u) == 0) codes[e >> 1] = (uint8_t)(c << 4);
        else codes[e >> 1] |= c;
    }
}

/* NF4 compress, block size 64 (nf4_impl.cpp:92-135).  scales[ceil(n/64)],
 * codes[ceil(n/2)]. */
ORACLE_API void oracle_nf4_compress(const float *x, uint64_t n, float *scales, uint8_t *codes) {
    const uint64_t bs = 64, nb = (n + bs - 1) / bs;
    int64_t b;
#pragma omp parallel for
    for (b = 0; b < (int64_t)nb; ++b) {
        const uint64_t start = (uint64_t)b * bs;
        const uint64_t remain = (start + bs <= n) ? bs : (n - start);
        const float m = block_absmax(x, start, remain);
        const float scale = (m > 0.0f) ? m : 1.0f;
        scales[b] = scale;
        encode_block(x, start, remain, 1.0f / scale, codes);
    }
}

/* NF4 decompress (nf4_impl.cpp:137-164): out = scale_b * level[code]. */
ORACLE_API void oracle_nf4_decompress(const float *scales, const uint8_t *codes, uint64_t n,
                                      float *out) {
    const uint64_t bs = 64, nb = (n + bs - 1) / bs;
    int64_t b;
#pragma omp parallel for
    for (b = 0; b < (int64_t)nb; ++b) {
        const uint64_t start = (uint64_t)b * bs;
        const uint64_t remain = (start + bs <= n) ? bs : (n - start);
        float s = scales[b];
        if (s == 0.0f || !isfinite(s)) s = 1.0f;
        for (uint64_t i = 0; i < remain; ++i) {
            const uint64_t e = start + i;
            const uint8_t p = codes[e >> 1];
            const uint8_t c = (e & 1u) ? (uint8_t)(p & 0xF) : (uint8_t)(p >> 4);
            out[e] = s * kLevels[c & 0xF];
        }
    }
}

/* FP8 E4M3 encode as the reference writes it (nf4_dq_impl.cpp:83-112):
 * non-finite -> +-448, clamp to 448, frexpf split, round-half-even mantissa,
 * sub-normal branch clamps the mantissa to 7. */
ORACLE_API uint8_t oracle_e4m3_encode(float x) {
    if (!isfinite(x)) x = (x < 0.0f) ? -448.0f : 448.0f;
    const int sign = signbit(x) ? 1 : 0;
    float ax = fabsf(x);
    if (ax == 0.0f) return (uint8_t)(sign << 7);
    if (ax > 448.0f) ax = 448.0f;
    int e2;
    const float mant = frexpf(ax, &e2);
    int ef = e2 - 1 + 7;
    if (ef <= 0) {
        int mf = (int)lrintf(ax * 512.0f);
        if (mf > 7) mf = 7;
        return (uint8_t)((sign << 7) | (mf & 0x7));
    }
    int mf = (int)lrintf(((mant * 2.0f) - 1.0f) * 8.0f);
    if (mf > 7) {
        mf = 0;
        ef += 1;
    }
    if (ef >= 16) {
        ef = 15;
        mf = 7;
    }
    return (uint8_t)((sign << 7) | ((ef & 0xF) << 3) | (mf & 0x7));
}

/* FP8 E4M3 decode (nf4_dq_impl.cpp:114-129); code 0x7F decodes to 480. */
ORACLE_API float oracle_e4m3_decode(uint8_t v) {
    const int sign = (v >> 7) & 1, ef = (v >> 3) & 0xF, mf = v & 7;
    float r;
    if (ef == 0) r = ((float)mf / 8.0f) * ldexpf(1.0f, 1 - 7);
    else r = (1.0f + (float)mf / 8.0f) * ldexpf(1.0f, ef - 7);
    return sign ? -r : r;
}

/* NF4_DQ compress (nf4_dq_impl.cpp:162-242): per-block absmax (zero block ->
 * 1), one global dq = max/448 (max over finite block scales; 0 -> 1), E4M3
 * code of absmax/dq per block, effective scale dq*E4M3^-1(code) (0 or
 * non-finite -> 1), then NF4 encode with its reciprocal. */
ORACLE_API void oracle_nf4dq_compress(const float *x, uint64_t n, float *dq_out,
                                      uint8_t *scale_codes, uint8_t *codes) {
    const uint64_t bs = 64, nb = (n + bs - 1) / bs;
    float *absmax = (float *)malloc(nb * sizeof(float));
    int64_t b;
#pragma omp parallel for
    for (b = 0; b < (int64_t)nb; ++b) {
        const uint64_t start = (uint64_t)b * bs;
        const uint64_t remain = (start + bs <= n) ? bs : (n - start);
        const float m = block_absmax(x, start, remain);
        absmax[b] = (m > 0.0f) ? m : 1.0f;
    }
    /* choose_dq_scale, nf4_dq_impl.cpp:150-160 */
    float gmax = 0.0f;
    for (uint64_t i = 0; i < nb; ++i) {
        const float v = absmax[i];
        if (!isfinite(v)) continue;
        const float a = fabsf(v);
        if (a > gmax) gmax = a;
    }
    float dq = (gmax == 0.0f) ? 1.0f : gmax / 448.0f;
    if (dq == 0.0f) dq = 1.0f;
    *dq_out = dq;
#pragma omp parallel for
    for (b = 0; b < (int64_t)nb; ++b) {
        const uint64_t start = (uint64_t)b * bs;
        const uint64_t remain = (start + bs <= n) ? bs : (n - start);
        const uint8_t sc = oracle_e4m3_encode(absmax[b] / dq);
        scale_codes[b] = sc;
        float s = dq * oracle_e4m3_decode(sc);
        if (s == 0.0f || !isfinite(s)) s = 1.0f;
        encode_block(x, start, remain, 1.0f / s, codes);
    }
    free(absmax);
}

/* NF4_DQ decompress (nf4_dq_impl.cpp:244-275): out = (dq*E4M3^-1(s_b)) * level.
 * The global dq is first replaced by 1 when it is 0 or not finite: the device
 * decoder on the bitsqz_llm path does that (quantization_cuda.cu:322-325),
 * the legacy CPU decoder does not; the two agree for every dq the encoders
 * write (a positive finite value), and only a loaded object can carry
 * another. */
ORACLE_API void oracle_nf4dq_decompress(float dq, const uint8_t *scale_codes,
                                        const uint8_t *codes, uint64_t n, float *out) {
    const uint64_t bs = 64, nb = (n + bs - 1) / bs;
    int64_t b;
    if (dq == 0.0f || !isfinite(dq)) dq = 1.0f;
#pragma omp parallel for
    for (b = 0; b < (int64_t)nb; ++b) {
        const uint64_t start = (uint64_t)b * bs;
        const uint64_t remain = (start + bs <= n) ? bs : (n - start);
        float s = dq * oracle_e4m3_decode(scale_codes[b]);
        if (s == 0.0f || !isfinite(s)) s = 1.0f;
        for (uint64_t i = 0; i < remain; ++i) {
            const uint64_t e = start + i;
            const uint8_t p = codes[e >> 1];
            const uint8_t c = (e & 1u) ? (uint8_t)(p & 0xF) : (uint8_t)(p >> 4);
            out[e] = s * kLevels[c & 0xF];
        }
    }
}

/* Batch helpers for tests. */
ORACLE_API void oracle_nf4_code_batch(const float *v, uint64_t n, uint8_t *out) {
    int64_t i;
#pragma omp parallel for
    for (i = 0; i < (int64_t)n; ++i) out[i] = oracle_nf4_code(v[i]);
}

ORACLE_API void oracle_e4m3_encode_batch(const float *v, uint64_t n, uint8_t *out) {
    int64_t i;
#pragma omp parallel for
    for (i = 0; i < (int64_t)n; ++i) out[i] = oracle_e4m3_encode(v[i]);
}

/* Exhaustive sweep of the NF4 code function over the bit patterns
 * [lo, hi) (hi exclusive, 64-bit so the full 2^32 range fits): writes a
 * 16-bin histogram and an order-independent checksum (sum over patterns of
 * code * (pattern mod 65521)).  Used to pin the device code function
 * against this one over all 2^32 floats without shipping 4 GiB. */
ORACLE_API void oracle_nf4_code_sweep(uint64_t lo, uint64_t hi, uint64_t *hist16,
                                      uint64_t *checksum) {
    uint64_t h[16] = {0};
    uint64_t cs = 0;
#pragma omp parallel
    {
        uint64_t hl[16] = {0};
        uint64_t csl = 0;
        int64_t p;
#pragma omp for
        for (p = (int64_t)lo; p < (int64_t)hi; ++p) {
            const uint32_t bits = (uint32_t)p;
            float f;
            memcpy(&f, &bits, 4);
            const uint8_t c = oracle_nf4_code(f);
            hl[c]++;
            csl += (uint64_t)c * (uint64_t)(bits % 65521u);
        }
#pragma omp critical
        {
            for (int i = 0; i < 16; ++i) h[i] += hl[i];
            cs += csl;
        }
    }
    for (int i = 0; i < 16; ++i) hist16[i] = h[i];
    *checksum = cs;
}

/* Per-row top-k (topk_cuda_utils.cuh:51-93 + topk_cuda.cu:186-201): keys are
 * |x| with NaN -> -inf; CUB's segmented radix sort is stable, so sorting each
 * row descending by key keeps equal keys in ascending column order.  That is
 * exactly a sort by (key desc, column asc), which qsort gives with the column
 * as a tie break.  Writes the first k columns and the signed source values. */
typedef struct {
    float key;
    uint16_t col;
} key_col_t;

static int cmp_key_col(const void *a, const void *b) {
    const key_col_t *x = (const key_col_t *)a, *y = (const key_col_t *)b;
    if (x->key > y->key) return -1;
    if (x->key < y->key) return 1;
    return (x->col < y->col) ? -1 : (x->col > y->col);
}

ORACLE_API void oracle_topk_rows(const float *x, uint32_t rows, uint32_t cols, uint32_t k,
                                 uint16_t *indices, float *values) {
    int64_t r;
#pragma omp parallel for
    for (r = 0; r < (int64_t)rows; ++r) {
        key_col_t *kc = (key_col_t *)malloc((size_t)cols * sizeof(key_col_t));
        const float *row = x + (uint64_t)r * cols;
        for (uint32_t c = 0; c < cols; ++c) {
            float key = fabsf(row[c]);
            if (isnan(key)) key = -INFINITY;
            kc[c].key = key;
            kc[c].col = (uint16_t)c;
        }
        qsort(kc, cols, sizeof(key_col_t), cmp_key_col);
        for (uint32_t j = 0; j < k; ++j) {
            indices[(uint64_t)r * k + j] = kc[j].col;
            values[(uint64_t)r * k + j] = row[kc[j].col];
        }
        free(kc);
    }
}

/* topk_compute_num_topk_columns (topk_cuda.cu:53-69): returns -1 for an
 * invalid ratio (the reference throws). */
ORACLE_API int oracle_topk_num_columns(uint16_t cols, float ratio) {
    if (cols == 0) return 0;
    if (!(ratio >= 0.0f && ratio <= 1.0f)) return -1;
    const float raw = (float)cols * ratio;
    uint16_t k = (uint16_t)roundf(raw);
    if (k > cols) k = cols;
    else if (k == 0 && ratio > 0.0f) k = 1;
    return (int)k;
}

/* Counts the finite floats with |v| < 2 in the bit-pattern range [lo, hi)
 * where the threshold rule code = #{c : v >= T[c]} disagrees with the
 * reference's linear scan (oracle_nf4_code).  Pins the device code
 * function's shortcut over every input it is used for. */
ORACLE_API uint64_t oracle_nf4_threshold_mismatches(const float *T, uint64_t lo, uint64_t hi) {
    uint64_t bad = 0;
    int64_t p;
#pragma omp parallel for reduction(+ : bad)
    for (p = (int64_t)lo; p < (int64_t)hi; ++p) {
        const uint32_t bits = (uint32_t)p;
        float v;
        memcpy(&v, &bits, 4);
        if (!(fabsf(v) < 2.0f)) continue;
        unsigned c = 0;
        for (int i = 0; i < 15; ++i) c += (v >= T[i]) ? 1u : 0u;
        if (c != oracle_nf4_code(v)) ++bad;
    }
    return bad;
}

/* Counts the floats with |v| < 2 in [lo, hi) where the 256-bin table rule of
 * the device NF4 code function (bin b = clamp(int((v + 1) * 128), 0, 255),
 * code = lo[b] + (v >= thr[b]), lo[b] = #{T_i <= -1 + b/128}, thr[b] the
 * threshold inside bin b or +inf) disagrees with the reference's linear scan.
 * The table is built with the same float arithmetic as the device. */
ORACLE_API uint64_t oracle_nf4_table_mismatches(const float *T, uint64_t lo, uint64_t hi) {
    float thr[256];
    unsigned lowc[256];
    for (int b = 0; b < 256; ++b) {
        const float e0 = -1.0f + (float)b / 128.0f, e1 = -1.0f + (float)(b + 1) / 128.0f;
        unsigned c = 0;
        float t = INFINITY;
        for (int i = 0; i < 15; ++i) {
            c += (T[i] <= e0) ? 1u : 0u;
            if (T[i] > e0 && T[i] < e1) t = T[i];
        }
        thr[b] = t;
        lowc[b] = c;
    }
    uint64_t bad = 0;
    int64_t p;
#pragma omp parallel for reduction(+ : bad)
    for (p = (int64_t)lo; p < (int64_t)hi; ++p) {
        const uint32_t bits = (uint32_t)p;
        float v;
        memcpy(&v, &bits, 4);
        if (!(fabsf(v) < 2.0f)) continue;
        int b = (int)((v + 1.0f) * 128.0f);
        b = b < 0 ? 0 : (b > 255 ? 255 : b);
        const unsigned c = lowc[b] + ((v >= thr[b]) ? 1u : 0u);
        if (c != oracle_nf4_code(v)) ++bad;
    }
    return bad;
}
