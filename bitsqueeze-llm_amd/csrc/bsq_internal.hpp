// Internal declarations shared by the HIP kernels and the host runtime of the
// MI355X (gfx950) bitsqz_llm library.  Nothing here is part of the public ABI
// (include/bitsqz_llm.hpp, include/bitsqz_llm_c.h).
#pragma once

#include <hip/hip_runtime.h>

#include <cstddef>
#include <cstdint>
#include <stdexcept>
#include <string>

namespace bsq {

// ---------------------------------------------------------------------------
// constants of the packed format (reference
// modules/quantization_cuda/include/quantization_cuda/quantization_cuda.cuh:10-13,
// src/bitsqz_llm.cu:25-29)
// ---------------------------------------------------------------------------
constexpr uint64_t kQuantBlock = 64;
constexpr float kE4M3Max = 448.0f;
constexpr uint32_t kQuantMagic = 0x51544355u;
constexpr uint16_t kQuantVersion = 1u;
constexpr int kMethodNF4DQ = 10;
constexpr int kMethodNF4 = 11;
constexpr int kMethodNone = -1;

constexpr uint32_t kFlagSvd = 1u << 0;
constexpr uint32_t kFlagOutlier = 1u << 1;
constexpr uint32_t kFlagError = 1u << 2;

// Exact decision thresholds of the NF4 nearest-code search.  For a finite v
// with |v| < 2 the reference's linear scan (first index minimising
// |fl(v - L[i])|, quantization_cuda.cu:43-58) returns #{c : v >= kNF4Thr[c]}.
// Each threshold is the smallest float at which the scan moves from code c to
// c + 1; they were found by bisection over float bit patterns and the identity
// is checked over every float with |v| < 2 by the CPU test suite.
#define BSQ_NF4_THRESHOLDS                                                          \
    {-0.848096371f, -0.610632896f, -0.45999524f, -0.33967942f, -0.234607399f,      \
     -0.137911722f, -0.0455250144f, 0.0397901535f, 0.120255254f, 0.203521267f,     \
     0.292013794f, 0.389312565f, 0.501663446f, 0.64278698f, 0.861478448f}
#define BSQ_NF4_THRESHOLD_BITS                                                      \
    {0xbf591cd8u, 0xbf1c5270u, 0xbeeb847fu, 0xbeadea76u, 0xbe703cecu, 0xbe0d38bbu,  \
     0xbd3a7870u, 0x3d22fb00u, 0x3df64863u, 0x3e5067e1u, 0x3e9582d5u, 0x3ec753fau,  \
     0x3f006d04u, 0x3f248db0u, 0x3f5c89dau}

// NF4 code book (reference quantization_cuda.cu:20-37).
#define BSQ_NF4_LEVELS                                                              \
    {-1.0f, -0.6961928009986877f, -0.5250730514526367f, -0.39491748809814453f,     \
     -0.28444138169288635f, -0.18477343022823334f, -0.09105003625154495f, 0.0f,    \
     0.07958029955625534f, 0.16093020141124725f, 0.24611230194568634f,             \
     0.33791524171829224f, 0.44070982933044434f, 0.5626170039176941f,              \
     0.7229568362236023f, 1.0f}

// ---------------------------------------------------------------------------
// error handling: internal code throws, the ABI layer catches
// ---------------------------------------------------------------------------
struct Error : std::runtime_error {
    using std::runtime_error::runtime_error;
};

[[noreturn]] void fail(const std::string &msg);
// Sets the message bsq_last_error() returns on this thread ("" clears it).
void set_last_error(const char *msg);
void hip_check(hipError_t e, const char *what);

#define BSQ_HIP(call) ::bsq::hip_check((call), #call)
#define BSQ_REQUIRE(cond, msg)            \
    do {                                  \
        if (!(cond)) ::bsq::fail(msg);    \
    } while (0)

__host__ __device__ inline uint64_t ceil_div(uint64_t a, uint64_t b) { return (a + b - 1) / b; }

typedef float f32x4 __attribute__((ext_vector_type(4)));

// ---------------------------------------------------------------------------
// kernel launchers (all asynchronous on `stream`)
// ---------------------------------------------------------------------------

// NF4 (method 11): scales_f32[ceil(n/64)], codes[ceil(n/2)].
// NF4_DQ (method 10): scales_u8[ceil(n/64)], *dq_out, codes; `gmax_scratch`
// is one device uint32 used for the global maximum.  A non-null `flags_reset`
// (one device uint32) is set to 0 by the encode kernel.  A non-null `sel`
// (n % 64 == 0) is a selection bitmap over x (byte j, bit i = element
// 8 j + i): flagged elements are encoded as 0 (x minus its separated
// outliers, without a residual copy).
void launch_quant_encode(const float *x, uint64_t n, int method, float *scales_f32,
                         uint8_t *scales_u8, float *dq_out, uint8_t *codes,
                         uint32_t *gmax_scratch, hipStream_t stream, uint32_t *flags_reset = nullptr,
                         const uint8_t *sel = nullptr);
// NF4_DQ global scale input: *gmax = bits of the largest block absmax of x
// (the first pass of launch_quant_encode; `codes` is scratch here, at least
// ceil(n / 2) bytes), or, from per-row maxima, of row_gmax[0 .. rows).
void launch_nf4dq_gmax(const float *x, uint64_t n, uint8_t *codes, uint32_t *gmax, hipStream_t stream);
void launch_rows_gmax(const float *row_gmax, uint32_t rows, uint32_t *gmax, hipStream_t stream);
// NF4_DQ encode whose global max of the block absmax is already known per row
// (row_gmax[0 .. rows), from the outlier separation): the encode pass, whose
// workgroups reduce the maxima themselves when rows <= kInlineGmaxRows and
// rows % 4 == 0 (else one small reduce launch first); the same bytes as
// launch_quant_encode.
void launch_quant_encode_dq_rows(const float *x, uint64_t n, const float *row_gmax, uint32_t rows,
                                 uint8_t *scales_u8, float *dq_out, uint8_t *codes, uint32_t *gmax_scratch,
                                 hipStream_t stream, const uint8_t *sel = nullptr);
void launch_quant_decode(uint64_t n, int method, const float *scales_f32,
                         const uint8_t *scales_u8, const float *dq, const uint8_t *codes,
                         float *out, hipStream_t stream);
// Decode of a rows x cols direct section fused with the decompress's top-k
// scatter (error set idx0 / val0 gated by *gate0's error flag when gate0 is
// given, then the outlier set idx1 / val1; k per row, in-row indices, those
// >= cols skipped): the same bytes as launch_quant_decode followed by
// launch_topk_scatter, one workgroup and one LDS row per matrix row.
constexpr uint32_t kDecodeRowsMaxCols = 32768;
bool quant_decode_rows_supported(uint32_t rows, uint32_t cols);
void launch_quant_decode_rows(uint32_t rows, uint32_t cols, int method, const float *scales_f32,
                              const uint8_t *scales_u8, const float *dq, const uint8_t *codes,
                              const uint16_t *idx0, const float *val0, uint32_t k0, const uint32_t *gate0,
                              const uint16_t *idx1, const float *val1, uint32_t k1, float *out,
                              hipStream_t stream);
void launch_nf4_code_batch(const float *v, uint64_t n, uint8_t *codes, hipStream_t stream);
void launch_e4m3_encode_batch(const float *v, uint64_t n, uint8_t *codes, hipStream_t stream);
void launch_e4m3_decode_batch(const uint8_t *c, uint64_t n, float *v, hipStream_t stream);
// Histogram (16 bins) + checksum sum(code * (bits % 65521)) of the NF4 code of
// every float bit pattern in [lo, hi).
void launch_nf4_code_sweep(uint64_t lo, uint64_t hi, unsigned long long *hist16,
                           unsigned long long *checksum, hipStream_t stream);

// Top-k.  Value sources for the per-row selection.
enum class TopkSource : int {
    Dense = 0,        // v = a[r, c]
    DenseMinusNF4 = 1,  // v = a[r, c] - dequant_nf4(...)[r, c]
    DenseMinusNF4DQ = 2,
    DenseMinusDense = 3,  // v = a[r, c] - b[r, c]
    // a is first encoded (NF4 / NF4_DQ, written to enc_*), then
    // v = a[r, c] - dequant(that encoding)[r, c]: the direct section's
    // encode and its error pass in one read of a
    EncodeNF4 = 4,
    EncodeNF4DQ = 5,
};
struct TopkArgs {
    const float *a = nullptr;         // row-major rows x cols
    const float *b = nullptr;         // DenseMinusDense subtrahend
    const float *scales_f32 = nullptr;  // NF4 block scales of the subtrahend
    const uint8_t *scales_u8 = nullptr; // NF4_DQ block scale codes
    const float *dq = nullptr;          // NF4_DQ global scale
    const uint8_t *codes = nullptr;     // packed nibbles of the subtrahend
    uint32_t rows = 0, cols = 0, k = 0;
    uint16_t *indices = nullptr;      // rows x k
    float *values = nullptr;          // rows x k
    float *residual = nullptr;        // optional: a with the selected entries zeroed
    uint32_t *flags = nullptr;        // optional: set to kFlagError if any |v| > FLT_EPSILON (the word holds 0 or kFlagError)
    // optional, with `residual`: row_gmax[r] = max over the residual's
    // 64-element blocks of row r of the block's largest sanitised |value|
    // (1 for an all-zero block), the per-row part of NF4_DQ's global scale
    float *row_gmax = nullptr;
    TopkSource source = TopkSource::Dense;
    // written 0 by the kernel before anything else reads it (the compress
    // flags word: the separation clears it instead of a memset launch)
    uint32_t *flags_reset = nullptr;
    // Encode sources: the section's codes (two per byte, element 2j in the
    // high nibble), block scales, and for NF4_DQ the bits of the largest
    // block absmax (input) and the raw global scale (written by row 0)
    uint8_t *enc_codes = nullptr;
    float *enc_scales_f32 = nullptr;
    uint8_t *enc_scales_u8 = nullptr;
    const uint32_t *enc_gmax = nullptr;
    float *enc_dq_out = nullptr;
    // EncodeNF4DQ, in place of enc_gmax: the per-row maxima of a separation
    // (row_gmax above; enc_gmax_rows of them, a multiple of 4 up to
    // kInlineGmaxRows, 16-byte aligned), reduced by every workgroup itself
    const float *enc_row_gmax = nullptr;
    uint32_t enc_gmax_rows = 0;
    // separation without a residual (Dense source, the register-resident
    // kernel, cols % 64 == 0): bit (r * cols + c) of sel_bits (32-bit words,
    // bit i of word w = element 32 w + i) is set when column c of row r is
    // selected, i.e. zeroed in the residual a caller would otherwise read
    uint32_t *sel_bits = nullptr;
    // Encode sources: the input is `a` with the entries flagged in enc_sel
    // (a sel_bits bitmap of the same shape) read as 0
    const uint32_t *enc_sel = nullptr;
    // Dense source: the input is read again right after this pass, so its
    // loads allocate in the caches (otherwise they are non-temporal)
    bool keep_input = false;
};
// Most per-row maxima the fused NF4_DQ encode reduces in every workgroup
// (TopkArgs::enc_row_gmax): four 16-byte loads per lane.
constexpr uint32_t kInlineGmaxRows = 4096;
// True when the fused encode + top-k pass (TopkSource::EncodeNF4 / EncodeNF4DQ)
// serves this shape: the register-resident kernel's shapes with cols % 64 == 0.
bool topk_encode_supported(uint32_t rows, uint32_t cols, uint32_t k, const float *a, const uint8_t *codes);
// True when the separation of k columns per row from `a` can write the
// selection bitmap (TopkArgs::sel_bits) and the per-row block maxima instead
// of a residual.
bool topk_selbits_supported(uint32_t rows, uint32_t cols, uint32_t k, const float *a);
// Returns true when row_gmax was requested and written (the register-resident
// kernel on a Dense source with cols % 64 == 0); otherwise row_gmax is left
// alone and the caller computes the global scale itself.  flags_reset is
// honoured on every path (by a memset where the kernel does not take it).
bool launch_topk_select(const TopkArgs &args, hipStream_t stream);
// Largest k the single-workgroup LDS sort handles; larger k (up to the row
// length) is sorted in bands of this many ranks.
constexpr uint32_t kTopkMaxK = 8192;

// dense[r, idx[r*k + j]] (+)= val[r*k + j]; with two lists, list 0 is applied
// before list 1 row by row (the reference applies the error set, then the
// outlier set).  When `gate0` is not null, list 0 is applied only if the
// device word *gate0 has kFlagError set.
void launch_topk_scatter(const uint16_t *idx0, const float *val0, uint32_t k0,
                         const uint16_t *idx1, const float *val1, uint32_t k1, uint32_t rows,
                         uint32_t cols, float *dense, bool accumulate, hipStream_t stream,
                         const uint32_t *gate0 = nullptr);
// One list scatter-added at flat positions r * cols + idx (the reference's
// indexing, for indices >= cols in loaded objects); positions >= rows * cols
// are skipped.
void launch_topk_scatter_flat(const uint16_t *idx, const float *val, uint32_t k, uint32_t rows,
                              uint32_t cols, float *dense, hipStream_t stream);

}  // namespace bsq

namespace bsq {

// ---------------------------------------------------------------------------
// randomised low-rank SVD and reconstruction
// ---------------------------------------------------------------------------
struct SvdPlan;
// Workspace for rank-q SVD of a row-major m x n matrix with `niter` power
// iterations (q is clamped to [1, min(m, n)]).
SvdPlan *svd_plan_create(int m, int n, int q, int niter);
void svd_plan_destroy(SvdPlan *plan) noexcept;
int svd_plan_rank(const SvdPlan *plan);
// Device bytes of every buffer of such a plan, each rounded up to 256 bytes.
uint64_t svd_plan_arena_bytes(int m, int n, int q, int niter);
// svd_run on a plan carved from the library's fixed device scratch array (no
// device allocation; asynchronous on `stream`; fails for shapes whose plan
// exceeds svd_noalloc_scratch_bytes()).
void svd_run_noalloc(const float *A, int m, int n, int q, int niter, const float *sketch, uint64_t seed, float *U,
                     float *S, float *V, hipStream_t stream);
uint64_t svd_noalloc_scratch_bytes();
// U (m x q), S (q), V (n x q), all row-major.  `sketch` (min(m,n) x q,
// row-major, device) replaces the built-in Gaussian sketch when not null.
void svd_run(SvdPlan *plan, const float *A, const float *sketch, uint64_t seed, float *U, float *S, float *V,
             hipStream_t stream);
// out = U diag(S) V^T (m x n row-major), or minuend - U diag(S) V^T when
// `minuend` is not null.
void launch_reconstruct(const float *U, const float *S, const float *V, int m, int n, int k,
                        const float *minuend, float *out, hipStream_t stream);
// N(0, 1) draws: Philox4x32-10 counter-based generator + Box-Muller.
void launch_gaussian_fill(float *out, uint64_t n, uint64_t seed, hipStream_t stream);

int cu_count();

// Reconstruction from NF4 / NF4_DQ factors decoded inline (recon.hip): U
// (m x k) and V (n x k) are packed nibbles with their block scales (and the
// device dq of NF4_DQ), S is FP32; out = U diag(S) V^T, bit for bit what
// decoding the factors and launch_reconstruct give.  Supported for
// k % 64 == 0, 64 <= k <= kReconQMaxK and 16-byte aligned code arrays.
constexpr int kReconQMaxK = 512;
bool recon_q_supported(int m, int n, int k, const uint8_t *u_codes, const uint8_t *v_codes);
void launch_recon_q(int method, const uint8_t *u_codes, const float *u_scales_f32, const uint8_t *u_scales_u8,
                    const float *u_dq, const uint8_t *v_codes, const float *v_scales_f32, const uint8_t *v_scales_u8,
                    const float *v_dq, const float *S, int m, int n, int k, float *out, hipStream_t stream);

// Instrumentation (off unless started through the ABI): HIP events bracket
// the launches of each class below inside the pipelines, on the stream they
// run on.  0: the low-rank reconstruction GEMM; 1: the range finder's
// products A_w B and A_w^T B (with their split-K / stream-K reductions);
// 2: the outlier separation (top-k); 3: the error-correction top-k pass;
// 4: the direct section's encode (with its NF4_DQ global-scale reduce);
// 5: the direct section's decode (with the fused top-k scatter when it runs).
enum GemmTimerClass {
    kTimeReconstruct = 0,
    kTimeRangeFinder = 1,
    kTimeTopkOutlier = 2,
    kTimeTopkError = 3,
    kTimeDirectEncode = 4,
    kTimeDirectDecode = 5,
    kTimeClasses = 6
};
bool gemm_timer_on();
void gemm_timer_begin(int cls, hipStream_t stream);
void gemm_timer_end(int cls, hipStream_t stream);
template <class F>
void timed_launch(int cls, hipStream_t stream, F &&launch) {
    if (!gemm_timer_on()) {
        launch();
        return;
    }
    gemm_timer_begin(cls, stream);
    launch();
    gemm_timer_end(cls, stream);
}

}  // namespace bsq
