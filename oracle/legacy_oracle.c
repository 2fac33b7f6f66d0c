/*
 * Legacy CPU codecs of the reference -- TEST INFRASTRUCTURE ONLY.
 *
 * A plain-C restatement of the eleven formats behind the reference's legacy
 * dispatcher (legacy_modules/quantization/src/quantization.cpp:125-382) other
 * than NF4 / NF4_DQ (which bsq_oracle.c restates): Q8_0, Q4_0, Q2_K,
 * Q2_K_FAST, BF16, FP16, FP8, FP4, MXFP8, MXFP4, NVFP4.  It is the checker of
 * the HIP codecs in csrc/legacy.hip; only tests/, __graft_entry__.smoke() and
 * bench.py's cpu_baseline leg may load it.
 *
 * Each function works on the raw arrays of a format (the struct headers and
 * payload layout are written by oracle/legacy.py) and cites the reference
 * lines it follows.  The floating-point steps are the reference's own, in the
 * same order and with the same libm calls (lrintf, frexpf, ldexpf, log2f,
 * ceilf), compiled with -ffp-contract=off like the reference's x86-64 build
 * (which has no FMA), so results are bit-identical on an x86-64 host.
 *
 * Pinning: tests/test_legacy_oracle.py checks every encoder and decoder here
 * against the golden vectors in tests/golden/legacy_golden.npz (written by the
 * reference's legacy library compiled from its own sources, oracle/Makefile),
 * against that library directly where it is built, and against closed forms
 * (exact FP16 / BF16 round-to-nearest-even over all 2^32 inputs, the E2M1 /
 * E4M3 code tables, exact recovery of representable values).
 */
#include <math.h>
#include <stdint.h>
#include <stdlib.h>
#include <string.h>

#define ORACLE_API __attribute__((visibility("default")))

/* ------------------------------------------------------------------------- */
/* scalar conversions                                                         */
/* ------------------------------------------------------------------------- */

static uint32_t f2u(float f) {
    uint32_t u;
    memcpy(&u, &f, 4);
    return u;
}
static float u2f(uint32_t u) {
    float f;
    memcpy(&f, &u, 4);
    return f;
}

/* FP32 -> BF16 (datatype/bf16.hpp:44-60): NaN keeps its top bits with the
 * quiet bit forced; otherwise round to nearest even on the low 16 bits. */
ORACLE_API uint16_t oracle_bf16_from_f32(float f) {
    uint32_t u = f2u(f);
    if ((u & 0x7F800000u) == 0x7F800000u && (u & 0x007FFFFFu) != 0) return (uint16_t)((u >> 16) | 0x0040u);
    const uint32_t low = u & 0xFFFFu, odd = (u >> 16) & 1u;
    if (low > 0x8000u || (low == 0x8000u && odd)) u += 0x10000u;
    return (uint16_t)(u >> 16);
}

/* BF16 -> FP32 (bf16.hpp:27-42): the bits in the high half. */
ORACLE_API float oracle_bf16_to_f32(uint16_t b) { return u2f((uint32_t)b << 16); }

/* FP32 -> FP16 as the FP16 header computes it on an x86-64 build without
 * F16C (datatype/fp16/fp16.hpp:119-152, the portable branch): IEEE binary16
 * round to nearest even, overflow to infinity, NaN -> sign | 0x7E00.  Here by
 * integer arithmetic on the bit pattern. */
ORACLE_API uint16_t oracle_fp16_from_f32(float f) {
    const uint32_t u = f2u(f), sign = (u >> 16) & 0x8000u, a = u & 0x7FFFFFFFu;
    if (a > 0x7F800000u) return (uint16_t)(sign | 0x7E00u);  /* NaN */
    if (a >= 0x477FF000u) return (uint16_t)(sign | 0x7C00u); /* >= 65520: rounds to infinity */
    if (a >= 0x38800000u) {                                  /* normal half (>= 2^-14) */
        const uint32_t m = a - 0x38000000u;                   /* rebias 127 -> 15, mantissa intact */
        const uint32_t keep = m >> 13, rem = m & 0x1FFFu;
        const uint32_t r = keep + ((rem > 0x1000u || (rem == 0x1000u && (keep & 1u))) ? 1u : 0u);
        return (uint16_t)(sign | r);
    }
    if (a < 0x33000000u) return (uint16_t)sign;               /* < 2^-25: rounds to zero */
    /* subnormal half: value / 2^-24 rounded to nearest even */
    const uint32_t e = a >> 23, mant = (a & 0x7FFFFFu) | 0x800000u;
    const uint32_t shift = 126u - e;                          /* 14 .. 24 */
    const uint32_t keep = mant >> shift, rem = mant & ((1u << shift) - 1u), half = 1u << (shift - 1u);
    const uint32_t r = keep + ((rem > half || (rem == half && (keep & 1u))) ? 1u : 0u);
    return (uint16_t)(sign | r);
}

/* FP16 -> FP32 (fp16.hpp:73-95): exact; NaN payloads move up 13 bits with
 * the quiet bit set (the portable branch multiplies the widened pattern by
 * 2^-112, which quiets a signalling NaN). */
ORACLE_API float oracle_fp16_to_f32(uint16_t h) {
    const uint32_t sign = (uint32_t)(h & 0x8000u) << 16, e = (h >> 10) & 0x1Fu, m = h & 0x3FFu;
    if (e == 0x1Fu) return u2f(sign | 0x7F800000u | (m << 13) | (m ? 0x400000u : 0u));
    if (e != 0) return u2f(sign | ((e + 112u) << 23) | (m << 13));
    if (m == 0) return u2f(sign);
    float v = (float)m * 0x1.0p-24f; /* exact */
    return sign ? -v : v;
}

/* E4M3 encode of the legacy FP8 / MXFP8 / NVFP4 codecs (fp8_impl.cpp:51-82,
 * mxfp8_impl.cpp:56-87, nvfp4_impl.cpp:62-93; identical bodies): saturating
 * at 448, frexpf split, lrintf of the 3-bit mantissa, subnormal mantissa
 * clamped at 7. */
ORACLE_API uint8_t oracle_legacy_e4m3_encode(float x) {
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
        return (uint8_t)((sign << 7) | (mf & 7));
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
    return (uint8_t)((sign << 7) | ((ef & 0xF) << 3) | (mf & 7));
}

/* E4M3 decode (fp8_impl.cpp:84-101): no NaN code, 0x7F -> 480. */
ORACLE_API float oracle_legacy_e4m3_decode(uint8_t v) {
    const int sign = (v >> 7) & 1, ef = (v >> 3) & 0xF, mf = v & 7;
    float r;
    if (ef == 0)
        r = ((float)mf / 8.0f) * ldexpf(1.0f, 1 - 7);
    else
        r = (1.0f + (float)mf / 8.0f) * ldexpf(1.0f, ef - 7);
    return sign ? -r : r;
}

/* E2M1 levels (fp4_impl.cpp:54-70): 0, 0.5, 1, 1.5, 2, 3, 4, 6. */
static float e2m1_level(int idx) {
    const int ef = idx >> 1, mf = idx & 1;
    if (idx == 0) return 0.0f;
    if (ef == 0) return ((float)mf / 2.0f) * ldexpf(1.0f, 0);
    return (1.0f + (float)mf / 2.0f) * ldexpf(1.0f, ef - 1);
}

/* E2M1 encode (fp4_impl.cpp:72-95; same in mxfp4 / nvfp4): non-finite -> 6,
 * nearest level by linear scan with strict '<' (ties to the lower index). */
ORACLE_API uint8_t oracle_e2m1_encode(float x) {
    const int sign = signbit(x) ? 1 : 0;
    float ax = fabsf(x);
    if (ax == 0.0f) return (uint8_t)(sign << 3);
    if (!isfinite(ax)) ax = 6.0f;
    if (ax > 6.0f) ax = 6.0f;
    int best = 0;
    float best_err = fabsf(e2m1_level(0) - ax);
    for (int i = 1; i < 8; ++i) {
        const float err = fabsf(e2m1_level(i) - ax);
        if (err < best_err) {
            best_err = err;
            best = i;
        }
    }
    return (uint8_t)((sign << 3) | (best & 7));
}

/* E2M1 decode (fp4_impl.cpp:97-112). */
ORACLE_API float oracle_e2m1_decode(uint8_t v) {
    const float r = e2m1_level(v & 7);
    return ((v >> 3) & 1) ? -r : r;
}

/* MX shared exponent (mxfp8_impl.cpp:121-127 with 448, mxfp4_impl.cpp:123-128
 * with 6): ceil(log2(abs_max / max_norm)) narrowed to int8 through int32 (as
 * the x86-64 build converts). */
ORACLE_API int8_t oracle_mx_scale_exp(float abs_max, float max_norm) {
    if (abs_max <= 0.0f) return 0;
    const float t = abs_max / max_norm;
    if (t <= 0.0f) return 0;
    return (int8_t)(int32_t)ceilf(log2f(t));
}

/* ------------------------------------------------------------------------- */
/* block formats with one absmax scale per block                              */
/* ------------------------------------------------------------------------- */

static uint64_t nblocks(uint64_t n, uint64_t bs) { return (n + bs - 1) / bs; }

/* Q8_0, block 32 (q8_0_impl.cpp:65-95). */
ORACLE_API void oracle_q8_0_encode(const float *x, uint64_t n, float *scales, int8_t *q) {
    const uint64_t nb = nblocks(n, 32);
    for (uint64_t b = 0; b < nb; ++b) {
        const uint64_t s = b * 32, r = (s + 32 <= n) ? 32 : n - s;
        float amax = 0.0f;
        for (uint64_t i = 0; i < r; ++i) {
            const float v = fabsf(x[s + i]);
            if (v > amax) amax = v;
        }
        const float scale = (amax > 0.0f) ? (amax / 127.0f) : 0.0f;
        const float inv = (scale > 0.0f) ? (1.0f / scale) : 0.0f;
        scales[b] = scale;
        for (uint64_t i = 0; i < r; ++i) {
            long qi = lrintf(x[s + i] * inv);
            if (qi < -127) qi = -127;
            if (qi > 127) qi = 127;
            q[s + i] = (int8_t)qi;
        }
    }
}

/* q8_0_impl.cpp:106-116. */
ORACLE_API void oracle_q8_0_decode(const float *scales, const int8_t *q, uint64_t n, float *out) {
    for (uint64_t i = 0; i < n; ++i) out[i] = scales[i / 32] * (float)q[i];
}

/* Q4_0, block 32, signed 4-bit codes in [-7, 7], element 2j in the high
 * nibble of byte j (q4_0_impl.cpp:70-109). */
ORACLE_API void oracle_q4_0_encode(const float *x, uint64_t n, float *scales, uint8_t *q) {
    const uint64_t nb = nblocks(n, 32);
    for (uint64_t b = 0; b < nb; ++b) {
        const uint64_t s = b * 32, r = (s + 32 <= n) ? 32 : n - s;
        float amax = 0.0f;
        for (uint64_t i = 0; i < r; ++i) {
            const float v = fabsf(x[s + i]);
            if (v > amax) amax = v;
        }
        const float scale = (amax > 0.0f) ? (amax / 7.0f) : 0.0f;
        const float inv = (scale > 0.0f) ? (1.0f / scale) : 0.0f;
        scales[b] = scale;
        for (uint64_t i = 0; i < r; ++i) {
            long qi = lrintf(x[s + i] * inv);
            if (qi < -7) qi = -7;
            if (qi > 7) qi = 7;
            const uint8_t c = (uint8_t)qi & 0x0F;
            const uint64_t j = s + i;
            if ((j & 1) == 0)
                q[j / 2] = (uint8_t)(c << 4);
            else
                q[j / 2] = (uint8_t)(q[j / 2] | c);
        }
    }
}

/* q4_0_impl.cpp:121-135: the nibble sign-extended. */
ORACLE_API void oracle_q4_0_decode(const float *scales, const uint8_t *q, uint64_t n, float *out) {
    for (uint64_t i = 0; i < n; ++i) {
        const uint8_t c = (i & 1) ? (q[i / 2] & 0x0F) : (q[i / 2] >> 4);
        const int8_t sv = (int8_t)(uint8_t)(c << 4) >> 4;
        out[i] = scales[i / 32] * (float)sv;
    }
}

/* MXFP8, block 32, E4M3 elements over a power-of-two scale 2^e
 * (mxfp8_impl.cpp:129-160): elements divided by the scale. */
ORACLE_API void oracle_mxfp8_encode(const float *x, uint64_t n, int8_t *scales, uint8_t *q) {
    const uint64_t nb = nblocks(n, 32);
    for (uint64_t b = 0; b < nb; ++b) {
        const uint64_t s = b * 32, r = (s + 32 <= n) ? 32 : n - s;
        float amax = 0.0f;
        for (uint64_t i = 0; i < r; ++i) {
            float v = x[s + i];
            if (!isfinite(v)) v = 0.0f;
            const float av = fabsf(v);
            if (av > amax) amax = av;
        }
        const int8_t e = oracle_mx_scale_exp(amax, 448.0f);
        scales[b] = e;
        const float scale = ldexpf(1.0f, e);
        for (uint64_t i = 0; i < r; ++i) q[s + i] = oracle_legacy_e4m3_encode(x[s + i] / scale);
    }
}

/* mxfp8_impl.cpp:162-182. */
ORACLE_API void oracle_mxfp8_decode(const int8_t *scales, const uint8_t *q, uint64_t n, float *out) {
    for (uint64_t i = 0; i < n; ++i) out[i] = ldexpf(1.0f, scales[i / 32]) * oracle_legacy_e4m3_decode(q[i]);
}

/* MXFP4, block 32, E2M1 elements times 2^-e (mxfp4_impl.cpp:130-170): the
 * elements are multiplied by ldexpf(1, -e). */
ORACLE_API void oracle_mxfp4_encode(const float *x, uint64_t n, int8_t *scales, uint8_t *q) {
    const uint64_t nb = nblocks(n, 32);
    for (uint64_t b = 0; b < nb; ++b) {
        const uint64_t s = b * 32, r = (s + 32 <= n) ? 32 : n - s;
        float amax = 0.0f;
        for (uint64_t i = 0; i < r; ++i) {
            float v = x[s + i];
            if (!isfinite(v)) v = 0.0f;
            const float av = fabsf(v);
            if (av > amax) amax = av;
        }
        const int8_t e = oracle_mx_scale_exp(amax, 6.0f);
        scales[b] = e;
        const float inv = ldexpf(1.0f, -e);
        for (uint64_t i = 0; i < r; ++i) {
            const uint8_t c = oracle_e2m1_encode(x[s + i] * inv) & 0xF;
            const uint64_t j = s + i;
            if ((j & 1) == 0)
                q[j / 2] = (uint8_t)(c << 4);
            else
                q[j / 2] = (uint8_t)(q[j / 2] | c);
        }
    }
}

/* mxfp4_impl.cpp:185-207. */
ORACLE_API void oracle_mxfp4_decode(const int8_t *scales, const uint8_t *q, uint64_t n, float *out) {
    for (uint64_t i = 0; i < n; ++i) {
        const uint8_t c = (i & 1) ? (q[i / 2] & 0x0F) : (q[i / 2] >> 4);
        out[i] = ldexpf(1.0f, scales[i / 32]) * oracle_e2m1_decode(c);
    }
}

/* ------------------------------------------------------------------------- */
/* formats with one tensor-wide scale                                         */
/* ------------------------------------------------------------------------- */

/* Largest finite |x| (fp8_impl.cpp:103-114 choose_scale; the same loop in
 * fp4_impl.cpp:114-125 and nvfp4_impl.cpp:174-185). */
static float finite_absmax(const float *x, uint64_t n) {
    float amax = 0.0f;
    for (uint64_t i = 0; i < n; ++i) {
        const float v = x[i];
        if (!isfinite(v)) continue;
        const float av = fabsf(v);
        if (av > amax) amax = av;
    }
    return amax;
}

/* FP8 (fp8_impl.cpp:116-146): scale = absmax / 448 (1 when absmax is 0),
 * elements times 1/scale to E4M3. */
ORACLE_API void oracle_fp8_encode(const float *x, uint64_t n, float *scale_out, uint8_t *q) {
    const float amax = finite_absmax(x, n);
    float scale = (amax == 0.0f) ? 1.0f : amax / 448.0f;
    if (scale == 0.0f) scale = 1.0f;
    *scale_out = scale;
    const float inv = 1.0f / scale;
    for (uint64_t i = 0; i < n; ++i) q[i] = oracle_legacy_e4m3_encode(x[i] * inv);
}

/* fp8_impl.cpp:133-146 (decode: scale * value). */
ORACLE_API void oracle_fp8_decode(float scale, const uint8_t *q, uint64_t n, float *out) {
    for (uint64_t i = 0; i < n; ++i) out[i] = scale * oracle_legacy_e4m3_decode(q[i]);
}

/* FP4 (fp4_impl.cpp:127-172): scale = absmax / 6, E2M1 nibbles, element 2j
 * high.  (The reference's element-parallel loop writes each byte from two
 * iterations; this restates its single-thread result.) */
ORACLE_API void oracle_fp4_encode(const float *x, uint64_t n, float *scale_out, uint8_t *q) {
    const float amax = finite_absmax(x, n);
    float scale = (amax == 0.0f) ? 1.0f : amax / 6.0f;
    if (scale == 0.0f) scale = 1.0f;
    *scale_out = scale;
    const float inv = 1.0f / scale;
    for (uint64_t i = 0; i < n; ++i) {
        const uint8_t c = oracle_e2m1_encode(x[i] * inv) & 0xF;
        if ((i & 1) == 0)
            q[i / 2] = (uint8_t)(c << 4);
        else
            q[i / 2] = (uint8_t)(q[i / 2] | c);
    }
}

/* fp4_impl.cpp:155-172. */
ORACLE_API void oracle_fp4_decode(float scale, const uint8_t *q, uint64_t n, float *out) {
    for (uint64_t i = 0; i < n; ++i) {
        const uint8_t c = (i & 1) ? (q[i / 2] & 0x0F) : (q[i / 2] >> 4);
        out[i] = scale * oracle_e2m1_decode(c);
    }
}

/* NVFP4, block 16 (nvfp4_impl.cpp:174-238): tensor scale = absmax / 6;
 * block scale = E4M3 of (max over the block of |x / tensor_scale|, non-finite
 * quotients as 0) / 6, or of 1 when that is 0; elements
 * (x * (1 / tensor_scale)) * (1 / block_scale) to E2M1. */
ORACLE_API void oracle_nvfp4_encode(const float *x, uint64_t n, float *tscale_out, uint8_t *bscales,
                                    uint8_t *q) {
    const float amax = finite_absmax(x, n);
    const float ts = (amax == 0.0f) ? 1.0f : amax / 6.0f;
    *tscale_out = ts;
    const float inv_ts = 1.0f / ts;
    const uint64_t nb = nblocks(n, 16);
    for (uint64_t b = 0; b < nb; ++b) {
        const uint64_t s = b * 16, r = (s + 16 <= n) ? 16 : n - s;
        float bmax = 0.0f;
        for (uint64_t i = 0; i < r; ++i) {
            float v = x[s + i] / ts;
            if (!isfinite(v)) v = 0.0f;
            const float av = fabsf(v);
            if (av > bmax) bmax = av;
        }
        const float target = bmax / 6.0f;
        const uint8_t code = oracle_legacy_e4m3_encode((target > 0.0f) ? target : 1.0f);
        bscales[b] = code;
        const float inv_bs = 1.0f / oracle_legacy_e4m3_decode(code);
        for (uint64_t i = 0; i < r; ++i) {
            const uint8_t c = oracle_e2m1_encode(x[s + i] * inv_ts * inv_bs) & 0xF;
            const uint64_t j = s + i;
            if ((j & 1) == 0)
                q[j / 2] = (uint8_t)(c << 4);
            else
                q[j / 2] = (uint8_t)(q[j / 2] | c);
        }
    }
}

/* nvfp4_impl.cpp:253-275: (tensor_scale * block_scale) * value. */
ORACLE_API void oracle_nvfp4_decode(float ts, const uint8_t *bscales, const uint8_t *q, uint64_t n,
                                    float *out) {
    for (uint64_t i = 0; i < n; ++i) {
        const uint8_t c = (i & 1) ? (q[i / 2] & 0x0F) : (q[i / 2] >> 4);
        out[i] = (ts * oracle_legacy_e4m3_decode(bscales[i / 16])) * oracle_e2m1_decode(c);
    }
}

/* ------------------------------------------------------------------------- */
/* Q2_K / Q2_K_FAST: 256-element super-blocks of sixteen 16-element blocks    */
/* ------------------------------------------------------------------------- */

/* One super-block record (q2_k_impl.hpp:12-17): fp16 super_scale, fp16
 * super_min, 16 packed (min << 4 | scale) bytes, 64 bytes of 2-bit codes;
 * 84 bytes, little-endian. */
#define Q2K_BYTES 84

/* Weighted least-squares search of the block scale and minimum
 * (q2_k_impl.cpp:59-140): a first fit from the range, then 16 trial inverse
 * scales around 3 / (max - min), keeping the smallest weighted L1 error. */
static void q2k_fit(const float *w, const float *aw, float *scale, float *minv) {
    float mn = w[0], mx = w[0], sw = aw[0], sx = sw * w[0];
    for (int i = 1; i < 16; ++i) {
        if (w[i] < mn) mn = w[i];
        if (w[i] > mx) mx = w[i];
        sw += aw[i];
        sx += aw[i] * w[i];
    }
    if (mn > 0) mn = 0;
    if (mx == mn) {
        *minv = mn;
        *scale = 0.0f;
        return;
    }
    float iscale = 3.0f / (mx - mn);
    float best_scale = 1.0f / iscale, best_err = 0.0f;
    for (int i = 0; i < 16; ++i) {
        int l = (int)lrintf(iscale * (w[i] - mn));
        l = l < 0 ? 0 : (l > 3 ? 3 : l);
        const float d = fabsf(best_scale * (float)(uint8_t)l + mn - w[i]);
        best_err += aw[i] * d;
    }
    for (int is = 0; is <= 15; ++is) {
        iscale = (-0.5f + 0.1f * (float)is + 3.0f) / (mx - mn);
        float sl = 0, sl2 = 0, sxl = 0;
        uint8_t la[16];
        for (int i = 0; i < 16; ++i) {
            int l = (int)lrintf(iscale * (w[i] - mn));
            l = l < 0 ? 0 : (l > 3 ? 3 : l);
            la[i] = (uint8_t)l;
            sl += aw[i] * (float)l;
            sl2 += aw[i] * (float)l * (float)l;
            sxl += aw[i] * (float)l * w[i];
        }
        const float D = sw * sl2 - sl * sl;
        if (D > 0) {
            float ts = (sw * sxl - sx * sl) / D;
            float tm = (sl2 * sx - sl * sxl) / D;
            if (tm > 0) {
                tm = 0;
                ts = sxl / sl2;
            }
            float err = 0;
            for (int i = 0; i < 16; ++i) err += aw[i] * fabsf(ts * (float)la[i] + tm - w[i]);
            if (err < best_err) {
                best_err = err;
                best_scale = ts;
                mn = tm;
            }
        }
    }
    *scale = best_scale;
    *minv = mn;
}

/* Range fit of Q2_K_FAST (q2_k_fast_impl.cpp:6-22): min, then max of
 * (w - min), scale = that / 3. */
static void q2k_fit_fast(const float *w, float *scale, float *minv) {
    float mn = INFINITY, mx = -INFINITY;
    for (int i = 0; i < 16; ++i)
        if (w[i] < mn) mn = w[i];
    for (int i = 0; i < 16; ++i) {
        const float s = w[i] - mn;
        if (s > mx) mx = s;
    }
    *scale = mx / 3.0f;
    *minv = mn;
}

static void put_u16(uint8_t *p, uint16_t v) {
    p[0] = (uint8_t)v;
    p[1] = (uint8_t)(v >> 8);
}
static uint16_t get_u16(const uint8_t *p) { return (uint16_t)(p[0] | (p[1] << 8)); }

/* q2_k_impl.cpp:142-236 (fast = 0) and q2_k_fast_impl.cpp:24-125 (fast = 1):
 * the input zero-padded to a multiple of 256; per super-block the sixteen
 * block fits, 4-bit block scales against super_scale = max_scale / 15 and
 * signed 4-bit block minimums against super_min = max|min| / 7 (both stored
 * as FP16), then 2-bit codes of (x - min_j) / scale_j, byte l of each 32-byte
 * half holding elements l, l + 32, l + 64, l + 96 of that half. */
ORACLE_API void oracle_q2k_encode(const float *x, uint64_t n, int fast, uint8_t *sb_out) {
    const uint64_t nsb = (n + 255) / 256;
    for (uint64_t s = 0; s < nsb; ++s) {
        float xs[256];
        for (int i = 0; i < 256; ++i) {
            const uint64_t g = s * 256 + (uint64_t)i;
            xs[i] = g < n ? x[g] : 0.0f;
        }
        uint8_t *rec = sb_out + s * Q2K_BYTES, *bsc = rec + 4, *codes = rec + 20;
        float scales[16], mins[16], max_scale = -INFINITY, max_abs_min = 0.0f;
        for (int j = 0; j < 16; ++j) {
            if (fast) {
                q2k_fit_fast(xs + 16 * j, &scales[j], &mins[j]);
            } else {
                float aw[16];
                for (int i = 0; i < 16; ++i) aw[i] = fabsf(xs[16 * j + i]);
                q2k_fit(xs + 16 * j, aw, &scales[j], &mins[j]);
            }
            if (scales[j] > max_scale) max_scale = scales[j];
            if (fabsf(mins[j]) > max_abs_min) max_abs_min = fabsf(mins[j]);
        }
        uint16_t super_scale, super_min;
        if (max_scale > 0) {
            const float is = 15.0f / max_scale;
            for (int j = 0; j < 16; ++j) bsc[j] = (uint8_t)(int)lrintf(is * scales[j]);
            super_scale = oracle_fp16_from_f32(max_scale / 15.0f);
        } else {
            memset(bsc, 0, 16);
            super_scale = oracle_fp16_from_f32(0.0f);
        }
        if (max_abs_min > 0) {
            const float is = 7.0f / max_abs_min;
            for (int j = 0; j < 16; ++j) {
                int l = (int)lrintf(is * mins[j]);
                l = l < -8 ? -8 : (l > 7 ? 7 : l);
                bsc[j] = (uint8_t)(bsc[j] | ((l & 0xF) << 4));
            }
            super_min = oracle_fp16_from_f32(max_abs_min / 7.0f);
        } else {
            super_min = oracle_fp16_from_f32(0.0f);
        }
        put_u16(rec, super_scale);
        put_u16(rec + 2, super_min);
        uint8_t L[256];
        const float ss = oracle_fp16_to_f32(super_scale), sm = oracle_fp16_to_f32(super_min);
        for (int j = 0; j < 16; ++j) {
            const float ts = ss * (float)(bsc[j] & 0xF);
            const int8_t mq = (int8_t)(uint8_t)(bsc[j] >> 4);
            const float tm = sm * (float)((int8_t)(uint8_t)(mq << 4) >> 4);
            for (int i = 0; i < 16; ++i) {
                const float v = (ts > 0.0f) ? (xs[16 * j + i] - tm) / ts : 0.0f;
                int l = (int)lrintf(v);
                l = l < 0 ? 0 : (l > 3 ? 3 : l);
                L[16 * j + i] = (uint8_t)l;
            }
        }
        for (int h = 0; h < 2; ++h)
            for (int l = 0; l < 32; ++l) {
                const uint8_t *g = L + 128 * h + l;
                codes[32 * h + l] = (uint8_t)(g[0] | (g[32] << 2) | (g[64] << 4) | (g[96] << 6));
            }
    }
}

/* q2_k_impl.cpp:348-422: min_j + scale_j * code. */
ORACLE_API void oracle_q2k_decode(const uint8_t *sb, uint64_t n, float *out) {
    const uint64_t nsb = (n + 255) / 256;
    for (uint64_t s = 0; s < nsb; ++s) {
        const uint8_t *rec = sb + s * Q2K_BYTES, *bsc = rec + 4, *codes = rec + 20;
        const float ss = oracle_fp16_to_f32(get_u16(rec)), sm = oracle_fp16_to_f32(get_u16(rec + 2));
        float sc[16], mn[16];
        for (int j = 0; j < 16; ++j) {
            sc[j] = ss * (float)(bsc[j] & 0x0F);
            const int8_t mq = (int8_t)(uint8_t)(bsc[j] >> 4);
            mn[j] = sm * (float)((int8_t)(uint8_t)(mq << 4) >> 4);
        }
        for (int i = 0; i < 256; ++i) {
            const uint64_t g = s * 256 + (uint64_t)i;
            if (g >= n) break;
            const int h = i / 128, w = i % 128, l = w % 32, shift = 2 * (w / 32);
            const int c = (codes[32 * h + l] >> shift) & 3;
            out[g] = mn[i / 16] + sc[i / 16] * (float)c;
        }
    }
}

/* ------------------------------------------------------------------------- */
/* elementwise formats                                                        */
/* ------------------------------------------------------------------------- */

/* bf16_impl.cpp:44-73, fp16_impl.cpp:44-73. */
ORACLE_API void oracle_bf16_encode(const float *x, uint64_t n, uint16_t *q) {
    for (uint64_t i = 0; i < n; ++i) q[i] = oracle_bf16_from_f32(x[i]);
}
ORACLE_API void oracle_bf16_decode(const uint16_t *q, uint64_t n, float *out) {
    for (uint64_t i = 0; i < n; ++i) out[i] = oracle_bf16_to_f32(q[i]);
}
ORACLE_API void oracle_fp16_encode(const float *x, uint64_t n, uint16_t *q) {
    for (uint64_t i = 0; i < n; ++i) q[i] = oracle_fp16_from_f32(x[i]);
}
ORACLE_API void oracle_fp16_decode(const uint16_t *q, uint64_t n, float *out) {
    for (uint64_t i = 0; i < n; ++i) out[i] = oracle_fp16_to_f32(q[i]);
}

/* ------------------------------------------------------------------------- */
/* exhaustive sweeps (checksums over every input pattern in [lo, hi))         */
/* ------------------------------------------------------------------------- */

/* kind 0: FP16 of every float pattern; 1: BF16; 2: MX exponent with max 448;
 * 3: MX exponent with max 6 (patterns of positive finite floats only
 * contribute for 2 and 3).  Sum over patterns of (result + 1) * (pattern mod
 * 65521), mod 2^64. */
ORACLE_API uint64_t oracle_legacy_sweep(int kind, uint64_t lo, uint64_t hi) {
    uint64_t acc = 0;
    for (uint64_t p = lo; p < hi; ++p) {
        const float f = u2f((uint32_t)p);
        uint64_t r;
        switch (kind) {
            case 0: r = oracle_fp16_from_f32(f); break;
            case 1: r = oracle_bf16_from_f32(f); break;
            case 2: r = (uint8_t)oracle_mx_scale_exp(f, 448.0f); break;
            default: r = (uint8_t)oracle_mx_scale_exp(f, 6.0f); break;
        }
        acc += (r + 1) * (p % 65521u);
    }
    return acc;
}
