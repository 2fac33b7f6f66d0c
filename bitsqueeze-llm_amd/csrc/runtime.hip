// Host runtime of the bitsqz_llm compress / decompress path on MI355X.
//
// Implements the nine C++-linkage entry points of include/bitsqz_llm.hpp with
// the reference's semantics (src/bitsqz_llm.cu:765-1455): two process-global
// runtimes (compress, decompress) configured at initialisation, the same
// argument validation and 0/1 return convention, the same packed object
// (200-byte header + sections U, S, V or direct, then outlier, then error),
// and the same section / top-k / quantisation blob layouts.
//
// Unlike the reference, the whole compress pipeline is enqueued on one HIP
// stream with no host synchronisation until the payload is copied out, the
// sections are kept in per-section device buffers (so a device-resident
// caller can decode without touching the host), the residual is only
// materialised when outliers are separated, and the error matrix is never
// materialised on the direct path (the error top-k kernel computes
// residual - dequant(direct) on the fly).
#include "bitsqz_llm.hpp"
#include "bitsqz_llm_c.h"
#include "bsq_internal.hpp"

#include <algorithm>
#include <atomic>
#include <cmath>
#include <condition_variable>
#include <cstdlib>
#include <cstring>
#include <limits>
#include <malloc.h>
#include <memory>
#include <mutex>
#include <thread>
#include <vector>

namespace bsq {

void fail(const std::string &msg) { throw Error(msg); }

void hip_check(hipError_t e, const char *what) {
    if (e != hipSuccess) throw Error(std::string(what) + ": " + hipGetErrorString(e));
}

int cu_count() {
    static int n = 0;
    if (n == 0) {
        int dev = 0;
        BSQ_HIP(hipGetDevice(&dev));
        BSQ_HIP(hipDeviceGetAttribute(&n, hipDeviceAttributeMultiprocessorCount, dev));
        if (n <= 0) n = 256;
    }
    return n;
}

namespace {

thread_local std::string g_last_error;

// Host copies of the packed payload (pinned staging <-> the caller's block)
// split over a few persistent threads: one thread copies about 10-20 GB/s,
// and a fresh calloc block also takes a page fault per 4 KB on first touch,
// which threads take in parallel.  The caller's thread copies too; chunks of
// 1 MB are taken from the job's atomic counter.  Each job is its own object,
// held by every thread that works on it, so a late worker never touches the
// next job's counters.  Calls are serialised.
class CopyPool {
  public:
    static CopyPool &get() {
        static CopyPool pool;
        return pool;
    }
    void copy(void *dst, const void *src, size_t n) {
        if (n < 2 * kChunk || workers_.empty()) {
            if (src) std::memcpy(dst, src, n);
            else std::memset(dst, 0, n);
            return;
        }
        std::lock_guard<std::mutex> call(call_mu_);
        auto job = std::make_shared<Job>();
        job->dst = static_cast<uint8_t *>(dst);
        job->src = static_cast<const uint8_t *>(src);
        job->n = n;
        job->chunks = (n + kChunk - 1) / kChunk;
        {
            std::lock_guard<std::mutex> lk(mu_);
            job_ = job;
            ++seq_;
        }
        cv_.notify_all();
        work(*job);
        std::unique_lock<std::mutex> lk(job->mu);
        job->cv.wait(lk, [&] { return job->done.load() == job->chunks; });
    }
    ~CopyPool() {
        {
            std::lock_guard<std::mutex> lk(mu_);
            stop_ = true;
        }
        cv_.notify_all();
        for (auto &t : workers_) t.join();
    }

  private:
    static constexpr size_t kChunk = 1u << 20;
    struct Job {
        uint8_t *dst = nullptr;
        const uint8_t *src = nullptr;
        size_t n = 0, chunks = 0;
        std::atomic<size_t> next{0}, done{0};
        std::mutex mu;
        std::condition_variable cv;
    };
    CopyPool() {
        const unsigned hw = std::thread::hardware_concurrency();
        const unsigned n = std::min(7u, hw > 1 ? hw - 1 : 0u);
        for (unsigned i = 0; i < n; ++i) workers_.emplace_back([this] { loop(); });
    }
    static void work(Job &j) {
        size_t c;
        while ((c = j.next.fetch_add(1)) < j.chunks) {
            const size_t off = c * kChunk, len = std::min(kChunk, j.n - off);
            if (j.src) std::memcpy(j.dst + off, j.src + off, len);
            else std::memset(j.dst + off, 0, len);
            if (j.done.fetch_add(1) + 1 == j.chunks) {
                std::lock_guard<std::mutex> lk(j.mu);
                j.cv.notify_all();
            }
        }
    }
    void loop() {
        uint64_t seen = 0;
        for (;;) {
            std::shared_ptr<Job> job;
            {
                std::unique_lock<std::mutex> lk(mu_);
                cv_.wait(lk, [&] { return stop_ || seq_ != seen; });
                if (stop_) return;
                seen = seq_;
                job = job_;
            }
            work(*job);
        }
    }
    std::vector<std::thread> workers_;
    std::mutex mu_, call_mu_;
    std::condition_variable cv_;
    std::shared_ptr<Job> job_;
    uint64_t seq_ = 0;
    bool stop_ = false;
};

void host_copy(void *dst, const void *src, size_t n) { CopyPool::get().copy(dst, src, n); }
// zeroes (and so faults in) a fresh host block with the same threads
void host_touch(void *dst, size_t n) { CopyPool::get().copy(dst, nullptr, n); }

// Packed objects handed back through bitsqz_llm_free are kept for the next
// compress (at most two, 1 GiB in total, blocks of 1 MiB and more): a fresh
// calloc block of that size is mapped lazily and takes a page fault per
// 4 KB on first touch, which a reused block has already taken.  They are
// malloc blocks, so a caller that releases an object with free() instead
// stays correct (that block is simply not kept).
class BlockCache {
  public:
    static BlockCache &get() {
        static BlockCache cache;
        return cache;
    }
    // a kept block of n bytes or a little more, or null
    void *take(size_t n) {
        std::lock_guard<std::mutex> lock(mu_);
        for (size_t i = 0; i < blocks_.size(); ++i) {
            const size_t cap = blocks_[i].second;
            if (cap >= n && cap <= n + n / 2) {
                void *p = blocks_[i].first;
                bytes_ -= cap;
                blocks_.erase(blocks_.begin() + static_cast<std::ptrdiff_t>(i));
                return p;
            }
        }
        return nullptr;
    }
    // true when the block is kept (the caller frees it otherwise)
    bool put(void *p) {
        const size_t cap = malloc_usable_size(p);
        if (cap < kMinBytes) return false;
        std::lock_guard<std::mutex> lock(mu_);
        if (blocks_.size() >= kMaxBlocks || bytes_ + cap > kMaxBytes) return false;
        blocks_.emplace_back(p, cap);
        bytes_ += cap;
        return true;
    }
    ~BlockCache() {
        for (auto &b : blocks_) std::free(b.first);
    }

  private:
    static constexpr size_t kMinBytes = size_t{1} << 20, kMaxBytes = size_t{1} << 30, kMaxBlocks = 2;
    std::mutex mu_;
    std::vector<std::pair<void *, size_t>> blocks_;
    size_t bytes_ = 0;
};

void set_error(const char *msg) { g_last_error = msg ? msg : ""; }

template <typename T>
T *dev_alloc(uint64_t count) {
    if (count == 0) return nullptr;
    void *p = nullptr;
    BSQ_HIP(hipMalloc(&p, count * sizeof(T)));
    return static_cast<T *>(p);
}

template <typename T>
void dev_free(T *&p) noexcept {
    if (p) (void)hipFree(p);
    p = nullptr;
}

// One dense-or-quantised section (U, S, V or direct) in device memory.
struct Section {
    int method = kMethodNone;  // NONE -> FP32 storage
    uint64_t count = 0;
    float *dense = nullptr;       // FP32 values (the section itself, or its dequantised copy)
    float *scales_f32 = nullptr;  // NF4
    uint8_t *scales_u8 = nullptr; // NF4_DQ
    uint8_t *codes = nullptr;
    bool own_dense = false;

    uint64_t nblocks() const { return ceil_div(count, kQuantBlock); }
    uint64_t packed_size() const {
        if (method == kMethodNone) return count * 4;
        return 48 + (method == kMethodNF4 ? nblocks() * 4 : nblocks()) + (count + 1) / 2;
    }
    void alloc_quant() {
        if (method == kMethodNF4) scales_f32 = dev_alloc<float>(nblocks());
        else scales_u8 = dev_alloc<uint8_t>(nblocks());
        codes = dev_alloc<uint8_t>((count + 1) / 2);
    }
    void release() noexcept {
        if (own_dense) dev_free(dense);
        dense = nullptr;
        own_dense = false;
        dev_free(scales_f32);
        dev_free(scales_u8);
        dev_free(codes);
        method = kMethodNone;
        count = 0;
    }
};

struct TopkBuf {
    uint16_t capacity = 0;  // k of the runtime (topk_compute_num_topk_columns)
    uint16_t *idx = nullptr;
    float *val = nullptr;
    void release() noexcept {
        dev_free(idx);
        dev_free(val);
        capacity = 0;
    }
};

enum { SEC_U = 0, SEC_S = 1, SEC_V = 2, SEC_DIRECT = 3 };
enum { TK_OUTLIER = 0, TK_ERROR = 1 };

// meta block in device memory: flags word (kFlagError set on the device),
// NF4_DQ global scales of the four sections, NF4_DQ max scratch.
struct Meta {
    uint32_t flags;
    float dq[4];
    uint32_t gmax;
    uint32_t pad[2];
};

struct Runtime {
    bool initialized = false;
    bool compress = false;
    uint16_t rows = 0, cols = 0;
    float r_out = 0.0f, r_err = 0.0f;
    int svd_ranks = -1, svd_niters = 1;
    int q = 0;  // allocated rank (svd_allocated_rank)
    int uv_fmt = kMethodNone, s_fmt = kMethodNone, direct_fmt = kMethodNone;
    int input_location = BITSQZ_LLM_INPUT_DEVICE;
    bool quant_initialized = false;
    bool reconstruct_initialized = false;

    hipStream_t stream = nullptr;
    bool owns_stream = true;   // false: a lane's decompress runtime borrowing its compress stream
    bool host_path = true;     // false: device-resident only (no copy stream, no pinned staging)
    hipEvent_t ev[8] = {};
    // payload copies between HBM and the pinned staging run on their own
    // stream (default priority), ordered after their producers by events, so
    // they overlap the compute stream's remaining work
    hipStream_t copy_stream = nullptr;
    hipEvent_t cev[4] = {};
    float *d_stage = nullptr;     // HOST-input staging
    float *d_residual = nullptr;  // input with outliers zeroed
    float *d_err = nullptr;       // residual - U S V^T (SVD path with error top-k)
    float *d_row_gmax = nullptr;  // per-row NF4_DQ block maxima from the outlier separation
    hipEvent_t t_begin = nullptr, t_end = nullptr;  // bitsqz_llm_compress wall span (profile struct)
    Section sec[4];
    TopkBuf topk[2];
    Meta *meta = nullptr;
    SvdPlan *svd = nullptr;
    const float *sketch = nullptr;  // injected Gaussian sketch (test hook)
    // decompress-side staging for quantised sections (shared, like the reference's buffers)
    float *q_scales_f32 = nullptr;
    uint8_t *q_scales_u8 = nullptr;
    uint8_t *q_codes = nullptr;
    // last compress result, device-resident
    bsq_device_packed_t last{};
    // pinned host staging of the packed payload (largest payload the
    // configuration can produce, plus the Meta block): the sections move
    // between HBM and the host object through it at full link speed
    uint8_t *h_stage = nullptr;
    uint64_t h_stage_bytes = 0;

    void release() noexcept {
        if (stream) (void)hipStreamSynchronize(stream);
        if (copy_stream) (void)hipStreamSynchronize(copy_stream);
        if (h_stage) (void)hipHostFree(h_stage);
        for (auto &s : sec) s.release();
        for (auto &t : topk) t.release();
        dev_free(d_stage);
        dev_free(d_residual);
        dev_free(d_err);
        dev_free(d_row_gmax);
        dev_free(meta);
        dev_free(q_scales_f32);
        dev_free(q_scales_u8);
        dev_free(q_codes);
        if (svd) svd_plan_destroy(svd);
        svd = nullptr;
        for (auto &e : ev)
            if (e) (void)hipEventDestroy(e);
        for (auto &e : cev)
            if (e) (void)hipEventDestroy(e);
        if (t_begin) (void)hipEventDestroy(t_begin);
        if (t_end) (void)hipEventDestroy(t_end);
        if (stream && owns_stream) (void)hipStreamDestroy(stream);
        if (copy_stream) (void)hipStreamDestroy(copy_stream);
        *this = Runtime{};
    }
};

Runtime g_comp;
Runtime g_decomp;

// Plain 16-byte-per-lane copy: the known-size reference against which HBM
// counters of the other kernels are calibrated (bytes read = bytes written =
// 16 * n4).
__global__ void copy_f32x4_kernel(const float4 *__restrict__ src, float4 *__restrict__ dst, uint64_t n4) {
    for (uint64_t i = static_cast<uint64_t>(blockIdx.x) * blockDim.x + threadIdx.x; i < n4;
         i += static_cast<uint64_t>(gridDim.x) * blockDim.x)
        dst[i] = src[i];
}

// HIP-event bracketing of the GEMMs over the m x n matrix (gemm_timer_*,
// declared in bsq_internal.hpp): one event pair per timed launch, created on
// first use and reused afterwards.
struct KernelTimer {
    std::vector<hipEvent_t> ev;  // pairs: ev[2i] before, ev[2i+1] after
    size_t used = 0;             // pairs recorded since the last read
    double last_ms = 0.0;        // totals of the last read
    int last_launches = 0;
    void begin(hipStream_t st) {
        if (2 * used + 2 > ev.size()) {
            hipEvent_t a = nullptr, b = nullptr;
            // no system-scope fence: these only time kernels on this device
            BSQ_HIP(hipEventCreateWithFlags(&a, hipEventDisableSystemFence));
            if (hipEventCreateWithFlags(&b, hipEventDisableSystemFence) != hipSuccess) {
                (void)hipEventDestroy(a);
                fail("kernel timer: hipEventCreate failed");
            }
            ev.push_back(a);
            ev.push_back(b);
        }
        BSQ_HIP(hipEventRecord(ev[2 * used], st));
    }
    void end(hipStream_t st) {
        BSQ_HIP(hipEventRecord(ev[2 * used + 1], st));
        ++used;
    }
    void read() {
        double t = 0.0;
        for (size_t i = 0; i < used; ++i) {
            BSQ_HIP(hipEventSynchronize(ev[2 * i + 1]));
            float ms = 0.0f;
            BSQ_HIP(hipEventElapsedTime(&ms, ev[2 * i], ev[2 * i + 1]));
            t += ms;
        }
        last_ms = t;
        last_launches = static_cast<int>(used);
        used = 0;
    }
};
bool g_timer_on = false;
KernelTimer g_gemm_timer[kTimeClasses];

}  // namespace

void set_last_error(const char *msg) { set_error(msg); }

bool gemm_timer_on() { return g_timer_on; }
void gemm_timer_begin(int cls, hipStream_t stream) { g_gemm_timer[cls].begin(stream); }
void gemm_timer_end(int cls, hipStream_t stream) { g_gemm_timer[cls].end(stream); }

namespace {

bool ratio_is_valid(float r) { return std::isfinite(r) && r >= 0.0f && r <= 1.0f; }
bool method_is_valid(int m) { return m == kMethodNone || m == kMethodNF4 || m == kMethodNF4DQ; }
bool uses_quant(const Runtime &rt) {
    return rt.uv_fmt != kMethodNone || rt.s_fmt != kMethodNone || rt.direct_fmt != kMethodNone;
}

}  // namespace

// topk_compute_num_topk_columns (modules/topk_cuda/src/topk_cuda.cu:53-69).
uint16_t topk_num_columns(uint16_t cols, float ratio) {
    if (cols == 0) return 0;
    if (!(ratio >= 0.0f && ratio <= 1.0f)) fail("topk_ratio must be in [0, 1]");
    const float raw = static_cast<float>(cols) * ratio;
    uint16_t k = static_cast<uint16_t>(roundf(raw));
    if (k > cols) k = cols;
    else if (k == 0 && ratio > 0.0f) k = 1;
    return k;
}

namespace {

void init_topk(TopkBuf &t, uint16_t rows, uint16_t cols, float ratio) {
    t.capacity = topk_num_columns(cols, ratio);
    if (t.capacity == 0) return;
    const uint64_t n = static_cast<uint64_t>(rows) * t.capacity;
    t.idx = dev_alloc<uint16_t>(n);
    t.val = dev_alloc<float>(n);
}

void create_stream(Runtime &rt, hipStream_t borrowed = nullptr) {
    if (borrowed) {
        rt.stream = borrowed;
        rt.owns_stream = false;
    } else {
        BSQ_HIP(hipStreamCreateWithFlags(&rt.stream, hipStreamNonBlocking));
    }
    if (rt.host_path) BSQ_HIP(hipStreamCreateWithFlags(&rt.copy_stream, hipStreamNonBlocking));
    for (auto &e : rt.ev) BSQ_HIP(hipEventCreate(&e));
    for (auto &e : rt.cev) BSQ_HIP(hipEventCreateWithFlags(&e, hipEventDisableTiming));
    rt.meta = dev_alloc<Meta>(1);
    BSQ_HIP(hipMemsetAsync(rt.meta, 0, sizeof(Meta), rt.stream));
}

uint64_t quant_section_bytes(int method, uint64_t count) {
    if (method == kMethodNone) return count * 4;
    const uint64_t nb = ceil_div(count, kQuantBlock);
    return 48 + (method == kMethodNF4 ? nb * 4 : nb) + (count + 1) / 2;
}

// Largest payload of the runtime's configuration: its dense / quantised
// sections and both top-k blobs at full capacity.
uint64_t max_payload_bytes(const Runtime &rt) {
    const uint64_t rows = rt.rows, cols = rt.cols;
    uint64_t p = 0;
    if (rt.svd_ranks >= 1) {
        const uint64_t q = static_cast<uint64_t>(rt.q);
        p += quant_section_bytes(rt.uv_fmt, rows * q) + quant_section_bytes(rt.s_fmt, q) +
             quant_section_bytes(rt.uv_fmt, cols * q);
    } else {
        p += quant_section_bytes(rt.direct_fmt, rows * cols);
    }
    for (const auto &t : rt.topk)
        if (t.capacity) p += 8 + rows * t.capacity * 6;
    return p;
}

void alloc_host_stage(Runtime &rt) {
    rt.h_stage_bytes = ceil_div(max_payload_bytes(rt), 256) * 256 + 2 * sizeof(Meta);
    void *p = nullptr;
    BSQ_HIP(hipHostMalloc(&p, rt.h_stage_bytes, hipHostMallocDefault));
    rt.h_stage = static_cast<uint8_t *>(p);
}

// bitsqz_llm_compress_initialize body (src/bitsqz_llm.cu:785-885).
void compress_init(Runtime &rt, uint16_t rows, uint16_t cols, float r_out, float r_err, int svd_ranks,
                   int svd_niters, int uv, int s, int direct, int loc, bool host_path = true) {
    rt.host_path = host_path;
    rt.compress = true;
    rt.rows = rows;
    rt.cols = cols;
    rt.r_out = r_out;
    rt.r_err = r_err;
    rt.svd_ranks = svd_ranks;
    rt.svd_niters = svd_niters;
    rt.uv_fmt = uv;
    rt.s_fmt = s;
    rt.direct_fmt = direct;
    rt.input_location = loc;
    create_stream(rt);
    const uint64_t N = static_cast<uint64_t>(rows) * cols;
    const bool has_svd = svd_ranks >= 1;
    if (loc == BITSQZ_LLM_INPUT_HOST) rt.d_stage = dev_alloc<float>(N);
    rt.quant_initialized = uses_quant(rt);
    if (r_out > 0.0f) init_topk(rt.topk[TK_OUTLIER], rows, cols, r_out);
    if (r_err > 0.0f) init_topk(rt.topk[TK_ERROR], rows, cols, r_err);
    rt.d_residual = dev_alloc<float>(N);
    if (has_svd) {
        const int q = std::max(1, std::min(svd_ranks, static_cast<int>(std::min(rows, cols))));
        rt.q = q;
        rt.svd = svd_plan_create(rows, cols, q, svd_niters);
        const int fmts[3] = {uv, s, uv};
        const uint64_t counts[3] = {static_cast<uint64_t>(rows) * q, static_cast<uint64_t>(q),
                                    static_cast<uint64_t>(cols) * q};
        for (int i = 0; i < 3; ++i) {
            Section &sc = rt.sec[i];
            sc.method = fmts[i];
            sc.count = counts[i];
            sc.dense = dev_alloc<float>(sc.count);
            sc.own_dense = true;
            if (sc.method != kMethodNone) sc.alloc_quant();
        }
        rt.reconstruct_initialized = true;
        if (rt.topk[TK_ERROR].capacity > 0) rt.d_err = dev_alloc<float>(N);
    } else {
        Section &sc = rt.sec[SEC_DIRECT];
        sc.method = direct;
        sc.count = N;
        if (sc.method != kMethodNone) sc.alloc_quant();
        if (direct == kMethodNF4DQ && rt.topk[TK_OUTLIER].capacity > 0) rt.d_row_gmax = dev_alloc<float>(rows);
    }
    BSQ_HIP(hipEventCreate(&rt.t_begin));
    BSQ_HIP(hipEventCreate(&rt.t_end));
    if (rt.host_path) alloc_host_stage(rt);
    BSQ_HIP(hipStreamSynchronize(rt.stream));
    rt.initialized = true;
}

// bitsqz_llm_decompress_initialize body (src/bitsqz_llm.cu:887-979).
void decompress_init(Runtime &rt, uint16_t rows, uint16_t cols, float r_out, float r_err, int svd_ranks, int uv,
                     int s, int direct, hipStream_t borrowed = nullptr) {
    rt.host_path = borrowed == nullptr;
    rt.compress = false;
    rt.rows = rows;
    rt.cols = cols;
    rt.r_out = r_out;
    rt.r_err = r_err;
    rt.svd_ranks = svd_ranks;
    rt.svd_niters = 1;
    rt.uv_fmt = uv;
    rt.s_fmt = s;
    rt.direct_fmt = direct;
    create_stream(rt, borrowed);
    const uint64_t N = static_cast<uint64_t>(rows) * cols;
    if (svd_ranks >= 1) {
        rt.q = svd_ranks;
        const uint64_t counts[3] = {static_cast<uint64_t>(rows) * svd_ranks, static_cast<uint64_t>(svd_ranks),
                                    static_cast<uint64_t>(cols) * svd_ranks};
        for (int i = 0; i < 3; ++i) {
            rt.sec[i].count = counts[i];
            rt.sec[i].dense = dev_alloc<float>(counts[i]);
            rt.sec[i].own_dense = true;
        }
        rt.reconstruct_initialized = true;
    }
    if (uses_quant(rt)) {
        // shared staging sized for the whole matrix (allocate_bitsqz_device_buffers,
        // src/bitsqz_llm.cu:230-247)
        const uint64_t nb = ceil_div(N, kQuantBlock);
        rt.q_scales_f32 = dev_alloc<float>(nb);
        rt.q_scales_u8 = dev_alloc<uint8_t>(nb);
        rt.q_codes = dev_alloc<uint8_t>((N + 1) / 2);
        rt.quant_initialized = true;
    }
    if (r_out > 0.0f) init_topk(rt.topk[TK_OUTLIER], rows, cols, r_out);
    if (r_err > 0.0f) init_topk(rt.topk[TK_ERROR], rows, cols, r_err);
    if (rt.host_path) alloc_host_stage(rt);
    BSQ_HIP(hipStreamSynchronize(rt.stream));
    rt.initialized = true;
}

// stage events recorded by compress_device
enum : int { kNoEvents = 0, kCopyEvents = 1, kAllEvents = 2 };

// The device-resident compress pipeline (src/bitsqz_llm.cu:981-1247 without
// the host copies).  Everything is enqueued on rt.stream.
void compress_device(Runtime &rt, const float *d_in, bsq_device_packed_t *out, const int stage_events) {
    const hipStream_t st = rt.stream;
    // stage boundaries: the host path's copy stream waits on ev[1] (after
    // the separation), ev[3] (after the encode) and ev[6] (the end), and a
    // requested profile reports the spans of all of them.  Each record costs
    // the queue a few microseconds of idle time, so only those needed are
    // recorded (none on the device-resident path).
    auto mark = [&](int i) {
        if (stage_events == kAllEvents || (stage_events == kCopyEvents && (i == 1 || i == 3 || i == 6)))
            BSQ_HIP(hipEventRecord(rt.ev[i], st));
    };
    const uint32_t rows = rt.rows, cols = rt.cols;
    const uint64_t N = static_cast<uint64_t>(rows) * cols;
    bsq_device_packed_t P{};
    bitsqz_llm_array_t &H = P.header;
    H.num_rows = rt.rows;
    H.num_columns = rt.cols;
    H.num_elements = static_cast<uint32_t>(N);
    H.outlier_topk_ratio = rt.r_out;
    H.error_correction_topk_ratio = rt.r_err;
    H.svd_ranks = static_cast<int16_t>(rt.svd_ranks);
    H.svd_niters = static_cast<int16_t>(rt.svd_niters);
    H.svd_uv_format = static_cast<quantization_method_t>(rt.uv_fmt);
    H.svd_s_format = static_cast<quantization_method_t>(rt.s_fmt);
    H.quantization_only_format = static_cast<quantization_method_t>(rt.direct_fmt);
    uint32_t flags = 0;

    mark(0);

    // outlier separation (topk_separation, src/bitsqz_llm.cu:1045-1056)
    const float *residual = d_in;
    bool have_row_gmax = false;
    TopkBuf &to = rt.topk[TK_OUTLIER];
    TopkBuf &te = rt.topk[TK_ERROR];
    const bool has_svd = rt.svd_ranks >= 1;
    const Section &Dq = rt.sec[SEC_DIRECT];
    // a quantised direct section after the separation: the separation writes
    // a selection bitmap (one bit per element, in the residual buffer) and
    // the encode reads the input with the flagged entries as 0, instead of
    // writing the residual and reading it back
    const bool selbits = !has_svd && to.capacity > 0 && Dq.method != kMethodNone &&
                         topk_selbits_supported(rows, cols, to.capacity, d_in) &&
                         (te.capacity == 0 || topk_encode_supported(rows, cols, te.capacity, d_in, Dq.codes));
    uint32_t *sel = selbits ? reinterpret_cast<uint32_t *>(rt.d_residual) : nullptr;
    if (to.capacity > 0) {
        TopkArgs a;
        a.a = d_in;
        a.rows = rows;
        a.cols = cols;
        a.k = to.capacity;
        a.indices = to.idx;
        a.values = to.val;
        a.residual = selbits ? nullptr : rt.d_residual;
        a.sel_bits = sel;
        // the encode reads the input again right after: the separation's
        // loads allocate in the caches (the 256 MB last-level cache serves
        // part of the second read)
        a.keep_input = selbits;
        // the direct NF4_DQ section's global scale needs the largest block
        // absmax of the residual: the separation kernel reports it per row
        a.row_gmax = rt.d_row_gmax;
        a.flags_reset = &rt.meta->flags;  // cleared here instead of a memset launch
        timed_launch(kTimeTopkOutlier, st, [&] { have_row_gmax = launch_topk_select(a, st); });
        BSQ_REQUIRE(!selbits || have_row_gmax || Dq.method != kMethodNF4DQ,
                    "compress: the bitmap separation reports the row maxima");
        residual = selbits ? d_in : rt.d_residual;
        flags |= kFlagOutlier;
    }
    // without the separation the flags word is cleared by the direct quant
    // encode when that is the only kernel before the readers, else by a fill
    const bool encode_clears = to.capacity == 0 && !has_svd && te.capacity == 0 && Dq.method != kMethodNone;
    if (to.capacity == 0 && !encode_clears) BSQ_HIP(hipMemsetAsync(&rt.meta->flags, 0, sizeof(uint32_t), st));
    mark(1);

    if (has_svd) {
        flags |= kFlagSvd;
        H.effective_rank = static_cast<int16_t>(rt.q);
        Section &U = rt.sec[SEC_U], &S = rt.sec[SEC_S], &V = rt.sec[SEC_V];
        svd_run(rt.svd, residual, rt.sketch, 1241ULL, U.dense, S.dense, V.dense, st);
        mark(2);
        // quantise U, S, V, each dequantised in place afterwards
        // (append_quantized_section with d_dequantized_dst = the source,
        // src/bitsqz_llm.cu:1078-1139)
        for (int i = 0; i < 3; ++i) {
            Section &sc = rt.sec[i];
            if (sc.method == kMethodNone) continue;
            launch_quant_encode(sc.dense, sc.count, sc.method, sc.scales_f32, sc.scales_u8, &rt.meta->dq[i],
                                sc.codes, &rt.meta->gmax, st);
        }
        mark(3);
        for (int i = 0; i < 3; ++i) {
            Section &sc = rt.sec[i];
            if (sc.method == kMethodNone) continue;
            launch_quant_decode(sc.count, sc.method, sc.scales_f32, sc.scales_u8, &rt.meta->dq[i], sc.codes,
                                sc.dense, st);
        }
        mark(4);
        if (te.capacity > 0) {
            // reconstruct + subtract fused (src/bitsqz_llm.cu:1141-1163)
            timed_launch(kTimeReconstruct, st, [&] {
                launch_reconstruct(U.dense, S.dense, V.dense, rows, cols, rt.q, residual, rt.d_err, st);
            });
            mark(5);
            TopkArgs a;
            a.a = rt.d_err;
            a.rows = rows;
            a.cols = cols;
            a.k = te.capacity;
            a.indices = te.idx;
            a.values = te.val;
            a.flags = &rt.meta->flags;
            timed_launch(kTimeTopkError, st, [&] { launch_topk_select(a, st); });
        } else {
            mark(5);
        }
    } else {
        Section &D = rt.sec[SEC_DIRECT];
        mark(2);
        const bool fused = D.method != kMethodNone && te.capacity > 0 &&
                           topk_encode_supported(rows, cols, te.capacity, residual, D.codes);
        if (fused) {
            // the encode and the error pass in one read of the residual (or
            // of the input and the separation's bitmap): codes and block
            // scales, then the top-k of residual - dequant(codes)
            // (src/bitsqz_llm.cu:1171-1227)
            D.dense = nullptr;
            const bool dq = D.method == kMethodNF4DQ;
            timed_launch(kTimeDirectEncode, st, [&] {
                // the per-row maxima of a separation are reduced inside the
                // pass when there are few enough of them
                const bool inline_gmax = dq && have_row_gmax && rows <= kInlineGmaxRows && rows % 4 == 0;
                if (dq && !inline_gmax) {
                    if (have_row_gmax) launch_rows_gmax(rt.d_row_gmax, rows, &rt.meta->gmax, st);
                    else launch_nf4dq_gmax(residual, N, D.codes, &rt.meta->gmax, st);
                }
                TopkArgs a;
                a.a = residual;
                a.rows = rows;
                a.cols = cols;
                a.k = te.capacity;
                a.indices = te.idx;
                a.values = te.val;
                a.flags = &rt.meta->flags;
                a.source = dq ? TopkSource::EncodeNF4DQ : TopkSource::EncodeNF4;
                a.enc_codes = D.codes;
                a.enc_scales_f32 = D.scales_f32;
                a.enc_scales_u8 = D.scales_u8;
                if (inline_gmax) {
                    a.enc_row_gmax = rt.d_row_gmax;
                    a.enc_gmax_rows = rows;
                } else {
                    a.enc_gmax = &rt.meta->gmax;
                }
                a.enc_dq_out = &rt.meta->dq[SEC_DIRECT];
                a.enc_sel = sel;
                launch_topk_select(a, st);
            });
            mark(3);
            mark(4);
            mark(5);
        } else if (D.method != kMethodNone) {
            D.dense = nullptr;
            timed_launch(kTimeDirectEncode, st, [&] {
                const uint8_t *sel8 = reinterpret_cast<const uint8_t *>(sel);
                if (have_row_gmax && D.method == kMethodNF4DQ)
                    launch_quant_encode_dq_rows(residual, N, rt.d_row_gmax, rows, D.scales_u8,
                                                &rt.meta->dq[SEC_DIRECT], D.codes, &rt.meta->gmax, st, sel8);
                else
                    launch_quant_encode(residual, N, D.method, D.scales_f32, D.scales_u8, &rt.meta->dq[SEC_DIRECT],
                                        D.codes, &rt.meta->gmax, st, encode_clears ? &rt.meta->flags : nullptr,
                                        sel8);
            });
            mark(3);
            mark(4);
            mark(5);
            if (te.capacity > 0) {
                // error = residual - dequant(direct), computed inside the top-k
                // kernel (src/bitsqz_llm.cu:1183-1227)
                BSQ_REQUIRE(!selbits, "compress: the error pass reads a residual");
                TopkArgs a;
                a.a = residual;
                a.rows = rows;
                a.cols = cols;
                a.k = te.capacity;
                a.indices = te.idx;
                a.values = te.val;
                a.flags = &rt.meta->flags;
                a.codes = D.codes;
                if (D.method == kMethodNF4) {
                    a.source = TopkSource::DenseMinusNF4;
                    a.scales_f32 = D.scales_f32;
                } else {
                    a.source = TopkSource::DenseMinusNF4DQ;
                    a.scales_u8 = D.scales_u8;
                    a.dq = &rt.meta->dq[SEC_DIRECT];
                }
                timed_launch(kTimeTopkError, st, [&] { launch_topk_select(a, st); });
            }
        } else {
            // FP32 direct section: the residual itself (copied when it is the
            // caller's buffer, so the packed object owns its data)
            if (residual != rt.d_residual)
                BSQ_HIP(hipMemcpyAsync(rt.d_residual, residual, N * 4, hipMemcpyDeviceToDevice, st));
            D.dense = rt.d_residual;
            mark(3);
            mark(4);
            mark(5);
        }
    }
    mark(6);
    BSQ_HIP(hipGetLastError());

    // descriptors: offsets are final except that the error section's
    // presence is decided on the device (flags word)
    H.flags = flags;
    uint64_t off = 0;
    bitsqz_section_t *descs[6] = {&H.section_u, &H.section_s, &H.section_v, &H.section_direct,
                                  &H.section_outlier_topk, &H.section_error_topk};
    const int order[4] = {SEC_U, SEC_S, SEC_V, SEC_DIRECT};
    for (int i : order) {
        const Section &sc = rt.sec[i];
        const bool present = has_svd ? (i != SEC_DIRECT) : (i == SEC_DIRECT);
        if (!present) continue;
        bitsqz_section_t &d = *descs[i];
        d.storage = sc.method == kMethodNone ? BITSQZ_SECTION_FP32 : BITSQZ_SECTION_QUANT;
        d.size = sc.packed_size();
        d.offset = off;
        off += d.size;
        P.d_dense[i] = sc.method == kMethodNone ? sc.dense : nullptr;
        P.d_scales_f32[i] = sc.scales_f32;
        P.d_scales_u8[i] = sc.scales_u8;
        P.d_dq_scale[i] = sc.method == kMethodNF4DQ ? &rt.meta->dq[i] : nullptr;
        P.d_codes[i] = sc.codes;
        P.count[i] = sc.count;
    }
    if (flags & kFlagOutlier) {
        bitsqz_section_t &d = H.section_outlier_topk;
        d.storage = BITSQZ_SECTION_TOPK;
        d.size = 8 + static_cast<uint64_t>(rows) * to.capacity * 6;
        d.offset = off;
        off += d.size;
        P.d_topk_idx[0] = to.idx;
        P.d_topk_val[0] = to.val;
        P.topk_k[0] = to.capacity;
    }
    if (te.capacity > 0) {
        // present only if the device sets kFlagError
        bitsqz_section_t &d = H.section_error_topk;
        d.storage = BITSQZ_SECTION_TOPK;
        d.size = 8 + static_cast<uint64_t>(rows) * te.capacity * 6;
        d.offset = off;
        P.d_topk_idx[1] = te.idx;
        P.d_topk_val[1] = te.val;
        P.topk_k[1] = te.capacity;
    }
    P.d_flags = &rt.meta->flags;
    rt.last = P;
    *out = P;
}

// Decode into d_dst (src/bitsqz_llm.cu:1304-1393): dense part, then the
// error top-k, then the outlier top-k, scatter-added in that order.
void decompress_device(Runtime &rt, const bsq_device_packed_t &P, const bool has_error, float *d_dst,
                       hipStream_t st, const uint32_t *err_gate = nullptr, bool scatter = true) {
    const bitsqz_llm_array_t &H = P.header;
    const uint32_t rows = H.num_rows, cols = H.num_columns;
    const bool has_outlier = (H.flags & kFlagOutlier) != 0;
    const uint32_t ke = has_error ? P.topk_k[1] : 0, ko = has_outlier ? P.topk_k[0] : 0;
    if (H.flags & kFlagSvd) {
        const int q = static_cast<uint16_t>(H.effective_rank);
        // packed U and V: the reconstruction decodes them inline
        const bool fused = H.svd_uv_format != kMethodNone && !P.d_dense[SEC_U] && !P.d_dense[SEC_V] &&
                           recon_q_supported(rows, cols, q, P.d_codes[SEC_U], P.d_codes[SEC_V]);
        const float *dense[3];
        for (int i = 0; i < 3; ++i) {
            if (P.d_dense[i]) {
                dense[i] = P.d_dense[i];
            } else if (!(fused && i != SEC_S)) {
                Section &sc = rt.sec[i];  // decompress runtime's dense U / S / V
                const int method = (i == SEC_S) ? H.svd_s_format : H.svd_uv_format;
                launch_quant_decode(P.count[i], method, P.d_scales_f32[i], P.d_scales_u8[i], P.d_dq_scale[i],
                                    P.d_codes[i], sc.dense, st);
                dense[i] = sc.dense;
            } else {
                dense[i] = nullptr;
            }
        }
        if (fused) {
            timed_launch(kTimeReconstruct, st, [&] {
                launch_recon_q(H.svd_uv_format, P.d_codes[SEC_U], P.d_scales_f32[SEC_U], P.d_scales_u8[SEC_U],
                               P.d_dq_scale[SEC_U], P.d_codes[SEC_V], P.d_scales_f32[SEC_V], P.d_scales_u8[SEC_V],
                               P.d_dq_scale[SEC_V], dense[SEC_S], rows, cols, q, d_dst, st);
            });
        } else {
            timed_launch(kTimeReconstruct, st,
                       [&] { launch_reconstruct(dense[0], dense[1], dense[2], rows, cols, q, nullptr, d_dst, st); });
        }
    } else {
        const uint64_t N = static_cast<uint64_t>(rows) * cols;
        if (P.d_dense[SEC_DIRECT]) {
            BSQ_HIP(hipMemcpyAsync(d_dst, P.d_dense[SEC_DIRECT], N * 4, hipMemcpyDeviceToDevice, st));
        } else if (scatter && (ke > 0 || ko > 0) && quant_decode_rows_supported(rows, cols)) {
            // decode and both top-k sets in one pass over the rows
            timed_launch(kTimeDirectDecode, st, [&] {
                launch_quant_decode_rows(rows, cols, H.quantization_only_format, P.d_scales_f32[SEC_DIRECT],
                                         P.d_scales_u8[SEC_DIRECT], P.d_dq_scale[SEC_DIRECT], P.d_codes[SEC_DIRECT],
                                         P.d_topk_idx[1], P.d_topk_val[1], ke, err_gate, P.d_topk_idx[0],
                                         P.d_topk_val[0], ko, d_dst, st);
            });
            return;
        } else {
            timed_launch(kTimeDirectDecode, st, [&] {
                launch_quant_decode(N, H.quantization_only_format, P.d_scales_f32[SEC_DIRECT],
                                    P.d_scales_u8[SEC_DIRECT], P.d_dq_scale[SEC_DIRECT], P.d_codes[SEC_DIRECT], d_dst,
                                    st);
            });
        }
    }
    if (!scatter) return;
    launch_topk_scatter(P.d_topk_idx[1], P.d_topk_val[1], ke, P.d_topk_idx[0], P.d_topk_val[0], ko, rows, cols, d_dst,
                        true, st, err_gate);
}

// True when some index of the host top-k blob at `p` (num_topk_columns per
// row) is >= cols.  Such an index addresses a later row in the reference's
// scatter (topk_cuda_utils.cuh:132-149), which the row-local fused scatter
// does not reproduce.
bool topk_blob_has_wide_index(const uint8_t *p, uint64_t n, uint32_t cols) {
    const uint8_t *q = p + sizeof(uint16_t) * 4;  // the indices (the blob may sit at any byte offset)
    uint16_t chunk[4096];
    uint16_t mx = 0;
    for (uint64_t i0 = 0; i0 < n; i0 += 4096) {
        const uint64_t m = std::min<uint64_t>(4096, n - i0);
        std::memcpy(chunk, q + 2 * i0, m * 2);
        for (uint64_t i = 0; i < m; ++i) mx = chunk[i] > mx ? chunk[i] : mx;  // vectorised max
    }
    return n > 0 && mx >= cols;
}

// ---------------------------------------------------------------------------
// host payload: writer and validation
// ---------------------------------------------------------------------------
struct QuantHeader {  // quantization_cuda_packed_header_t (quantization_cuda.cuh:15-26)
    uint32_t magic;
    uint16_t version;
    uint16_t reserved0;
    int32_t method;
    uint32_t reserved1;
    uint64_t num_elements;
    uint64_t num_blocks;
    uint64_t block_size;
    float dq_scale;
    uint32_t reserved2;
};
static_assert(sizeof(QuantHeader) == 48, "quant header layout");
struct TopkHeader {  // topk_packed_header_t (topk_cuda.cuh:16-21)
    uint16_t num_rows, num_columns, num_topk_columns, reserved;
};
static_assert(sizeof(TopkHeader) == 8, "top-k header layout");
static_assert(sizeof(bitsqz_llm_array_t) == 200, "bitsqz_llm_array_t must be 200 bytes");
static_assert(offsetof(bitsqz_llm_array_t, section_u) == 48, "section_u offset");
static_assert(offsetof(bitsqz_llm_array_t, payload) == 192, "payload offset");

// The host packed object (src/bitsqz_llm.cu:1237-1277).  Every section part
// goes device -> pinned staging at its final payload offset, in three groups
// on the copy stream, each as soon as its producer has run: the outlier blob
// after the separation, the dense / quantised sections after the encode, the
// error blob (whose presence the device decides) after the last kernel.  The
// host fills the caller's calloc block group by group, so only the last
// group's copies follow the compute.
bitsqz_llm_array_t *assemble_host(Runtime &rt, const bsq_device_packed_t &P) {
    const hipStream_t cs = rt.copy_stream;
    bitsqz_llm_array_t H = P.header;
    const bitsqz_section_t *descs[6] = {&H.section_u, &H.section_s, &H.section_v, &H.section_direct,
                                        &H.section_outlier_topk, &H.section_error_topk};
    uint64_t full = 0;  // payload bytes with the error blob
    for (auto *d : descs)
        if (d->storage != BITSQZ_SECTION_NONE) full = std::max(full, d->offset + d->size);
    BSQ_REQUIRE(full + 2 * sizeof(Meta) <= rt.h_stage_bytes, "packed payload larger than the host staging");
    // the staging holds every part at its final payload offset, plus two
    // snapshots of the Meta block (dq scales after the encode, flags at the end)
    uint8_t *stage = rt.h_stage;
    Meta *meta_sec = reinterpret_cast<Meta *>(stage + rt.h_stage_bytes - 2 * sizeof(Meta));
    Meta *meta_end = reinterpret_cast<Meta *>(stage + rt.h_stage_bytes - sizeof(Meta));
    auto copy_topk = [&](int t) {
        const bitsqz_section_t &d = *descs[4 + t];
        if (d.storage == BITSQZ_SECTION_NONE) return;
        const uint64_t n = static_cast<uint64_t>(H.num_rows) * P.topk_k[t];
        BSQ_HIP(hipMemcpyAsync(stage + d.offset + 8, P.d_topk_idx[t], n * 2, hipMemcpyDeviceToHost, cs));
        BSQ_HIP(hipMemcpyAsync(stage + d.offset + 8 + n * 2, P.d_topk_val[t], n * 4, hipMemcpyDeviceToHost, cs));
    };
    auto section_method = [&](int i) {
        return (i == SEC_S) ? H.svd_s_format : (i == SEC_DIRECT ? H.quantization_only_format : H.svd_uv_format);
    };
    // group 0: the outlier blob, final once the separation has run (ev[1])
    BSQ_HIP(hipStreamWaitEvent(cs, rt.ev[1], 0));
    copy_topk(0);
    BSQ_HIP(hipEventRecord(rt.cev[0], cs));
    // group 1: U, S, V or the direct section, final after the encode (ev[3])
    BSQ_HIP(hipStreamWaitEvent(cs, rt.ev[3], 0));
    for (int i = 0; i < 4; ++i) {
        const bitsqz_section_t &d = *descs[i];
        if (d.storage == BITSQZ_SECTION_NONE) continue;
        uint8_t *dst = stage + d.offset;
        if (d.storage == BITSQZ_SECTION_FP32) {
            BSQ_HIP(hipMemcpyAsync(dst, P.d_dense[i], P.count[i] * 4, hipMemcpyDeviceToHost, cs));
            continue;
        }
        const int method = section_method(i);
        const uint64_t nb = ceil_div(P.count[i], kQuantBlock);
        const uint64_t ssz = method == kMethodNF4 ? nb * 4 : nb;
        const void *ssrc = method == kMethodNF4 ? static_cast<const void *>(P.d_scales_f32[i])
                                                : static_cast<const void *>(P.d_scales_u8[i]);
        BSQ_HIP(hipMemcpyAsync(dst + 48, ssrc, ssz, hipMemcpyDeviceToHost, cs));
        BSQ_HIP(hipMemcpyAsync(dst + 48 + ssz, P.d_codes[i], (P.count[i] + 1) / 2, hipMemcpyDeviceToHost, cs));
    }
    BSQ_HIP(hipMemcpyAsync(meta_sec, rt.meta, sizeof(Meta), hipMemcpyDeviceToHost, cs));
    BSQ_HIP(hipEventRecord(rt.cev[1], cs));
    // group 2: the error blob and the final flags, after the last kernel (ev[6])
    BSQ_HIP(hipStreamWaitEvent(cs, rt.ev[6], 0));
    copy_topk(1);
    BSQ_HIP(hipMemcpyAsync(meta_end, rt.meta, sizeof(Meta), hipMemcpyDeviceToHost, cs));
    BSQ_HIP(hipEventRecord(rt.cev[2], cs));

    // the host object, sized for every section (the error blob's presence is
    // decided last; a smaller object leaves the tail unused), filled group by
    // group while the device still works on the later ones
    void *raw = BlockCache::get().take(200 + full);
    const bool reused = raw != nullptr;
    if (!reused) raw = std::calloc(1, 200 + full);
    std::unique_ptr<void, void (*)(void *)> block(raw, std::free);
    BSQ_REQUIRE(block != nullptr, "calloc of the packed object failed");
    uint8_t *pl = static_cast<uint8_t *>(block.get()) + 200;
    // calloc maps a large block lazily: its pages are faulted in by several
    // threads while the copies above are still in flight, so the copies
    // below run without faults (a reused block has its pages already; every
    // byte of it up to the object's end is written below)
    if (!reused) host_touch(pl, full);
    auto put_topk = [&](int t) {
        const bitsqz_section_t &d = *descs[4 + t];
        if (d.storage == BITSQZ_SECTION_NONE) return;
        const TopkHeader th{H.num_rows, H.num_columns, P.topk_k[t], 0};
        std::memcpy(pl + d.offset, &th, sizeof(th));
        host_copy(pl + d.offset + 8, stage + d.offset + 8, d.size - 8);
    };
    BSQ_HIP(hipEventSynchronize(rt.cev[0]));
    put_topk(0);
    BSQ_HIP(hipEventSynchronize(rt.cev[1]));
    const Meta msec = *meta_sec;
    for (int i = 0; i < 4; ++i) {
        const bitsqz_section_t &d = *descs[i];
        if (d.storage == BITSQZ_SECTION_NONE) continue;
        if (d.storage == BITSQZ_SECTION_QUANT) {
            const int method = section_method(i);
            QuantHeader qh{};
            qh.magic = kQuantMagic;
            qh.version = kQuantVersion;
            qh.method = method;
            qh.num_elements = P.count[i];
            qh.num_blocks = ceil_div(P.count[i], kQuantBlock);
            qh.block_size = kQuantBlock;
            qh.dq_scale = method == kMethodNF4DQ ? msec.dq[i] : 0.0f;
            std::memcpy(pl + d.offset, &qh, sizeof(qh));
            host_copy(pl + d.offset + 48, stage + d.offset + 48, d.size - 48);
        } else {
            host_copy(pl + d.offset, stage + d.offset, d.size);
        }
    }
    BSQ_HIP(hipEventSynchronize(rt.cev[2]));
    const Meta mend = *meta_end;
    const bool err_present = P.topk_k[1] > 0 && (mend.flags & kFlagError);
    if (err_present) {
        H.flags |= kFlagError;
        put_topk(1);
    } else {
        // the error blob's space stays as calloc leaves it
        const bitsqz_section_t &d = *descs[5];
        if (reused && d.storage != BITSQZ_SECTION_NONE) host_copy(pl + d.offset, nullptr, d.size);
        H.section_error_topk = bitsqz_section_t{};
    }
    auto *buf = static_cast<bitsqz_llm_array_t *>(block.release());
    std::memcpy(buf, &H, sizeof(H));
    buf->payload = reinterpret_cast<uint8_t *>(buf) + 200;
    return buf;
}

// validate_section_bounds (src/bitsqz_llm.cu:319-332)
bool section_bounds_ok(const bitsqz_section_t &s, uint64_t payload_size) {
    if (s.storage == BITSQZ_SECTION_NONE) return s.size == 0;
    if (s.size == 0) return false;
    if (s.offset > payload_size) return false;
    if (s.size > payload_size - s.offset) return false;
    return s.storage == BITSQZ_SECTION_FP32 || s.storage == BITSQZ_SECTION_QUANT || s.storage == BITSQZ_SECTION_TOPK;
}

// validate_section_method_pair (src/bitsqz_llm.cu:617-631)
bool section_method_ok(const bitsqz_section_t &s, int method) {
    if (s.storage == BITSQZ_SECTION_NONE) return true;
    if (s.storage == BITSQZ_SECTION_FP32) return method == kMethodNone;
    if (s.storage == BITSQZ_SECTION_QUANT) return method != kMethodNone && method_is_valid(method);
    return false;
}

// topk_validate_packed_buffer (topk_cuda.cu:255-282)
bool topk_blob_ok(const uint8_t *p, uint64_t size, TopkHeader *out) {
    if (p == nullptr || size < sizeof(TopkHeader)) return false;
    TopkHeader h;
    std::memcpy(&h, p, sizeof(h));
    const uint64_t expected = 8 + static_cast<uint64_t>(h.num_rows) * h.num_topk_columns * 6;
    if (h.num_rows == 0 || h.num_columns == 0) return false;
    if (h.num_topk_columns > h.num_columns) return false;
    if (size != expected) return false;
    if (out) *out = h;
    return true;
}

// validate_topk_runtime_compatibility (src/bitsqz_llm.cu:633-652)
bool topk_runtime_ok(const TopkBuf &t, const bitsqz_llm_array_t *c, const bitsqz_section_t &s) {
    if (t.capacity == 0 || c == nullptr || c->payload == nullptr) return false;
    TopkHeader h;
    if (!topk_blob_ok(static_cast<const uint8_t *>(c->payload) + s.offset, s.size, &h)) return false;
    if (h.num_rows != c->num_rows || h.num_columns != c->num_columns) return false;
    return h.num_topk_columns <= t.capacity;
}

// validate_decompress_compatibility (src/bitsqz_llm.cu:654-761)
bool decompress_compatible(const Runtime &cfg, const bitsqz_llm_array_t *c) {
    if (c == nullptr || c->payload == nullptr) return false;
    if (c->num_rows == 0 || c->num_columns == 0 || c->num_elements == 0) return false;
    if (cfg.rows != c->num_rows || cfg.cols != c->num_columns) return false;
    if (c->num_elements != static_cast<uint32_t>(c->num_rows) * static_cast<uint32_t>(c->num_columns)) return false;
    const uint64_t packed = bitsqz_llm_get_packed_size(c);
    if (packed < sizeof(bitsqz_llm_array_t)) return false;
    const uint64_t payload = packed - sizeof(bitsqz_llm_array_t);
    const bitsqz_section_t secs[6] = {c->section_u, c->section_s, c->section_v, c->section_direct,
                                      c->section_outlier_topk, c->section_error_topk};
    for (const auto &s : secs)
        if (!section_bounds_ok(s, payload)) return false;
    const bool has_svd = c->flags & kFlagSvd, has_out = c->flags & kFlagOutlier, has_err = c->flags & kFlagError;
    if (!section_method_ok(c->section_u, c->svd_uv_format) || !section_method_ok(c->section_s, c->svd_s_format) ||
        !section_method_ok(c->section_v, c->svd_uv_format) ||
        !section_method_ok(c->section_direct, c->quantization_only_format))
        return false;
    auto has = [](const bitsqz_section_t &s) { return s.storage != BITSQZ_SECTION_NONE; };
    if (has_svd) {
        const uint16_t rank = static_cast<uint16_t>(c->effective_rank);
        if (rank == 0) return false;
        if (!cfg.reconstruct_initialized || cfg.svd_ranks != static_cast<int>(rank) ||
            cfg.q != static_cast<int>(rank))
            return false;
        if (!has(c->section_u) || !has(c->section_s) || !has(c->section_v) || has(c->section_direct)) return false;
    } else {
        if (c->effective_rank != 0) return false;
        if (!has(c->section_direct) || has(c->section_u) || has(c->section_s) || has(c->section_v)) return false;
    }
    const bool needs_quant = c->section_u.storage == BITSQZ_SECTION_QUANT ||
                             c->section_s.storage == BITSQZ_SECTION_QUANT ||
                             c->section_v.storage == BITSQZ_SECTION_QUANT ||
                             c->section_direct.storage == BITSQZ_SECTION_QUANT;
    if (needs_quant && !cfg.quant_initialized) return false;
    if (has_out) {
        if (c->section_outlier_topk.storage != BITSQZ_SECTION_TOPK ||
            !topk_runtime_ok(cfg.topk[TK_OUTLIER], c, c->section_outlier_topk))
            return false;
    } else if (has(c->section_outlier_topk)) {
        return false;
    }
    if (has_err) {
        if (c->section_error_topk.storage != BITSQZ_SECTION_TOPK ||
            !topk_runtime_ok(cfg.topk[TK_ERROR], c, c->section_error_topk))
            return false;
    } else if (has(c->section_error_topk)) {
        return false;
    }
    return true;
}

// quantization_cuda_validate_packed_buffer + the unpack checks
// (quantization_cuda.cu:691-734, 809-832)
bool quant_blob_ok(const uint8_t *p, uint64_t size, int method, uint64_t count, QuantHeader *out) {
    if (p == nullptr || size < sizeof(QuantHeader)) return false;
    QuantHeader h;
    std::memcpy(&h, p, sizeof(h));
    if (h.magic != kQuantMagic || h.version != kQuantVersion) return false;
    if (h.method != kMethodNF4 && h.method != kMethodNF4DQ) return false;
    if (h.num_elements == 0 || h.block_size != kQuantBlock) return false;
    if (h.num_blocks != ceil_div(h.num_elements, kQuantBlock)) return false;
    const uint64_t expected =
        48 + (h.method == kMethodNF4 ? h.num_blocks * 4 : h.num_blocks) + (h.num_elements + 1) / 2;
    if (size != expected) return false;
    if (h.method != method || h.num_elements != count) return false;
    if (out) *out = h;
    return true;
}

// H2D of a host packed object into the decompress runtime's buffers; fills a
// device descriptor for decompress_device.  Mirrors decode_section_to_device
// and topk_unpack_from_buffer (src/bitsqz_llm.cu:539-607, topk_cuda.cu:332-383).
void decompress_host(Runtime &rt, const bitsqz_llm_array_t *c, float *d_dst) {
    const hipStream_t st = rt.stream, cs = rt.copy_stream;
    // The caller's payload is pageable host memory.  Each section is copied by
    // the host into the pinned staging (same offset) and moves to the device
    // from there at full link speed; a section that does not fit the staging
    // (e.g. an FP32 direct section in a runtime configured for another path)
    // is copied from where it lies.  The dense sections go first, on the
    // compute stream; the top-k blobs follow on the copy stream while the
    // device decodes and reconstructs, and the scatter waits for them.
    const uint8_t *src = static_cast<const uint8_t *>(c->payload);
    const uint64_t stage_cap = rt.h_stage ? rt.h_stage_bytes - 2 * sizeof(Meta) : 0;
    auto staged = [&](const bitsqz_section_t &s) -> const uint8_t * {
        if (s.offset + s.size > stage_cap) return src;
        host_copy(rt.h_stage + s.offset, src + s.offset, s.size);
        return rt.h_stage;
    };
    // payload bytes [off, off + n) to the device through the staging in
    // pieces of 4 MB: each piece's H2D is issued as soon as the host has
    // staged it, so the link works while the host stages the next
    auto h2d_pieces = [&](void *dev, uint64_t off, uint64_t n, hipStream_t s) {
        if (off + n > stage_cap) {
            BSQ_HIP(hipMemcpyAsync(dev, src + off, n, hipMemcpyHostToDevice, s));
            return;
        }
        constexpr uint64_t kPiece = 4ull << 20;
        for (uint64_t q = 0; q < n; q += kPiece) {
            const uint64_t len = std::min(kPiece, n - q);
            host_copy(rt.h_stage + off + q, src + off + q, len);
            BSQ_HIP(hipMemcpyAsync(static_cast<uint8_t *>(dev) + q, rt.h_stage + off + q, len,
                                   hipMemcpyHostToDevice, s));
        }
    };
    bsq_device_packed_t P{};
    P.header = *c;
    const uint32_t rows = c->num_rows, cols = c->num_columns;
    const uint64_t N = static_cast<uint64_t>(rows) * cols;

    // top-k blobs: validated before anything is enqueued
    const bitsqz_section_t *tsec[2] = {&c->section_outlier_topk, &c->section_error_topk};
    const uint32_t tflag[2] = {kFlagOutlier, kFlagError};
    uint64_t tn[2] = {0, 0};
    bool tpresent[2] = {false, false}, wide = false;
    for (int t = 0; t < 2; ++t) {
        if (!(c->flags & tflag[t])) continue;
        BSQ_REQUIRE(rt.topk[t].capacity > 0, "top-k runtime missing");
        TopkHeader h;
        BSQ_REQUIRE(topk_blob_ok(src + tsec[t]->offset, tsec[t]->size, &h), "invalid top-k section");
        BSQ_REQUIRE(h.num_rows == rows && h.num_columns == cols && h.num_topk_columns <= rt.topk[t].capacity,
                    "top-k section incompatible with the runtime");
        tpresent[t] = true;
        tn[t] = static_cast<uint64_t>(rows) * h.num_topk_columns;
        P.d_topk_idx[t] = rt.topk[t].idx;
        P.d_topk_val[t] = rt.topk[t].val;
        P.topk_k[t] = h.num_topk_columns;
    }

    // Packed U and V of the SVD path stay packed for the reconstruction, which
    // decodes them inline, when both fit the shared staging side by side;
    // otherwise every section is decoded as soon as it arrives (the staging
    // is then shared).
    const uint64_t uq = (c->flags & kFlagSvd) ? static_cast<uint64_t>(rows) * static_cast<uint16_t>(c->effective_rank) : 0;
    const uint64_t vq = (c->flags & kFlagSvd) ? static_cast<uint64_t>(cols) * static_cast<uint16_t>(c->effective_rank) : 0;
    const uint64_t v_code_off = ceil_div(uq / 2, 256) * 256, v_scale_off = ceil_div(uq / kQuantBlock, 64) * 64;
    // a packed S is decoded at once, from behind V (U and V must stay intact)
    const uint64_t s_code_off = ceil_div(v_code_off + vq / 2, 256) * 256,
                   s_scale_off = ceil_div(v_scale_off + vq / kQuantBlock, 64) * 64;
    const uint64_t sq = (c->flags & kFlagSvd) ? static_cast<uint16_t>(c->effective_rank) : 0;
    const bool keep_packed = (c->flags & kFlagSvd) && c->svd_uv_format != kMethodNone && rt.quant_initialized &&
                             c->section_u.storage == BITSQZ_SECTION_QUANT &&
                             c->section_v.storage == BITSQZ_SECTION_QUANT &&
                             recon_q_supported(rows, cols, static_cast<uint16_t>(c->effective_rank), rt.q_codes,
                                               rt.q_codes + v_code_off) &&
                             s_code_off + (sq + 1) / 2 <= (N + 1) / 2 &&
                             s_scale_off + ceil_div(sq, kQuantBlock) <= ceil_div(N, kQuantBlock);
    auto stage_section = [&](int i, const bitsqz_section_t &s, int method, uint64_t count, float *dense_dst) {
        if (s.storage == BITSQZ_SECTION_FP32) {
            BSQ_REQUIRE(s.size == count * 4, "FP32 section size mismatch");
            h2d_pieces(dense_dst, s.offset, count * 4, st);
            P.d_dense[i] = dense_dst;
            P.count[i] = count;
            return;
        }
        BSQ_REQUIRE(s.storage == BITSQZ_SECTION_QUANT && method != kMethodNone, "bad quantised section");
        BSQ_REQUIRE(rt.quant_initialized, "quantisation runtime missing");
        QuantHeader h;
        BSQ_REQUIRE(quant_blob_ok(src + s.offset, s.size, method, count, &h), "invalid quantised section");
        const uint64_t nb = h.num_blocks;
        const uint64_t ssz = method == kMethodNF4 ? nb * 4 : nb;
        // the header and block scales staged at once, the codes piecewise
        const bitsqz_section_t head{s.offset, 48 + ssz, s.storage};
        const uint8_t *pl = staged(head);
        // packed U at the start of the staging, packed V after it
        const bool packed = keep_packed && (i == SEC_U || i == SEC_V);
        const uint64_t coff = !keep_packed ? 0 : (i == SEC_V ? v_code_off : (i == SEC_S ? s_code_off : 0));
        const uint64_t soff = !keep_packed ? 0 : (i == SEC_V ? v_scale_off : (i == SEC_S ? s_scale_off : 0));
        float *sc_f32 = rt.q_scales_f32 + soff;
        uint8_t *sc_u8 = rt.q_scales_u8 + soff, *codes = rt.q_codes + coff;
        void *sdst = method == kMethodNF4 ? static_cast<void *>(sc_f32) : static_cast<void *>(sc_u8);
        BSQ_HIP(hipMemcpyAsync(sdst, pl + s.offset + 48, ssz, hipMemcpyHostToDevice, st));
        h2d_pieces(codes, s.offset + 48 + ssz, (count + 1) / 2, st);
        if (method == kMethodNF4DQ)
            BSQ_HIP(hipMemcpyAsync(&rt.meta->dq[i], pl + s.offset + 40, 4, hipMemcpyHostToDevice, st));
        P.count[i] = count;
        if (packed) {
            P.d_dense[i] = nullptr;
            P.d_codes[i] = codes;
            P.d_scales_f32[i] = method == kMethodNF4 ? sc_f32 : nullptr;
            P.d_scales_u8[i] = method == kMethodNF4DQ ? sc_u8 : nullptr;
            P.d_dq_scale[i] = method == kMethodNF4DQ ? &rt.meta->dq[i] : nullptr;
            return;
        }
        // decode now (the staging buffers are shared between sections)
        launch_quant_decode(count, method, sc_f32, sc_u8, &rt.meta->dq[i], codes, dense_dst, st);
        P.d_dense[i] = dense_dst;
    };
    if (c->flags & kFlagSvd) {
        const uint16_t q = static_cast<uint16_t>(c->effective_rank);
        stage_section(SEC_U, c->section_u, c->svd_uv_format, static_cast<uint64_t>(rows) * q, rt.sec[SEC_U].dense);
        stage_section(SEC_S, c->section_s, c->svd_s_format, q, rt.sec[SEC_S].dense);
        stage_section(SEC_V, c->section_v, c->svd_uv_format, static_cast<uint64_t>(cols) * q, rt.sec[SEC_V].dense);
        decompress_device(rt, P, false, d_dst, st, nullptr, false);  // the reconstruction (scatter below)
    } else {
        stage_section(SEC_DIRECT, c->section_direct, c->quantization_only_format, N, d_dst);
        P.d_dense[SEC_DIRECT] = nullptr;  // already decoded into d_dst
    }

    // top-k blobs: host copy and H2D overlap the decode / reconstruction
    if (tpresent[0] || tpresent[1]) {
        for (int t = 0; t < 2; ++t) {
            if (!tpresent[t] || tn[t] == 0) continue;
            const uint8_t *pl = staged(*tsec[t]);
            BSQ_HIP(hipMemcpyAsync(rt.topk[t].idx, pl + tsec[t]->offset + 8, tn[t] * 2, hipMemcpyHostToDevice, cs));
            BSQ_HIP(hipMemcpyAsync(rt.topk[t].val, pl + tsec[t]->offset + 8 + tn[t] * 2, tn[t] * 4,
                                   hipMemcpyHostToDevice, cs));
            // the scatter's form (in-row or flat positions) from the copy just made
            wide = wide || topk_blob_has_wide_index(pl + tsec[t]->offset, tn[t], cols);
        }
        BSQ_HIP(hipEventRecord(rt.cev[3], cs));
        BSQ_HIP(hipStreamWaitEvent(st, rt.cev[3], 0));
    }
    const bool has_err = tpresent[1], has_out = tpresent[0];
    if (wide) {
        // the reference's two launches: the error set, then the outlier set
        // (src/bitsqz_llm.cu:1373-1387), each at flat positions
        if (has_err) launch_topk_scatter_flat(P.d_topk_idx[1], P.d_topk_val[1], P.topk_k[1], rows, cols, d_dst, st);
        if (has_out) launch_topk_scatter_flat(P.d_topk_idx[0], P.d_topk_val[0], P.topk_k[0], rows, cols, d_dst, st);
    } else {
        launch_topk_scatter(P.d_topk_idx[1], P.d_topk_val[1], has_err ? P.topk_k[1] : 0, P.d_topk_idx[0],
                            P.d_topk_val[0], has_out ? P.topk_k[0] : 0, rows, cols, d_dst, true, st);
    }
    BSQ_HIP(hipStreamSynchronize(st));
}

template <typename F>
int guarded(F &&f) {
    try {
        f();
        set_error("");
        return 0;
    } catch (const std::exception &e) {
        set_error(e.what());
        return 1;
    } catch (...) {
        set_error("unknown error");
        return 1;
    }
}

}  // namespace
}  // namespace bsq

using namespace bsq;

// ===========================================================================
// C++-linkage ABI (include/bitsqz_llm.hpp)
// ===========================================================================

int bitsqz_llm_compress_initialize(uint16_t num_rows, uint16_t num_columns, float outlier_topk_ratio,
                                   float error_correction_topk_ratio, int svd_ranks, int svd_niters,
                                   quantization_method_t svd_uv_format, quantization_method_t svd_s_format,
                                   quantization_method_t quantization_only_format,
                                   bitsqz_llm_input_location_t input_location) {
    if (num_rows == 0 || num_columns == 0) return 1;
    if (!ratio_is_valid(outlier_topk_ratio) || !ratio_is_valid(error_correction_topk_ratio)) return 1;
    if (!method_is_valid(svd_uv_format) || !method_is_valid(svd_s_format) ||
        !method_is_valid(quantization_only_format))
        return 1;
    if (input_location != BITSQZ_LLM_INPUT_HOST && input_location != BITSQZ_LLM_INPUT_DEVICE) return 1;
    if (svd_niters < 1) return 1;
    bitsqz_llm_compress_release();
    const int rc = guarded([&] {
        compress_init(g_comp, num_rows, num_columns, outlier_topk_ratio, error_correction_topk_ratio, svd_ranks,
                      svd_niters,
                      svd_uv_format, svd_s_format, quantization_only_format, input_location);
    });
    if (rc != 0) {
        const std::string msg = g_last_error;
        bitsqz_llm_compress_release();
        set_error(msg.c_str());
    }
    return rc;
}

void bitsqz_llm_compress_release() { g_comp.release(); }

int bitsqz_llm_decompress_initialize(uint16_t num_rows, uint16_t num_columns, float outlier_topk_ratio,
                                     float error_correction_topk_ratio, int svd_ranks,
                                     quantization_method_t svd_uv_format, quantization_method_t svd_s_format,
                                     quantization_method_t quantization_only_format) {
    if (num_rows == 0 || num_columns == 0) return 1;
    if (!ratio_is_valid(outlier_topk_ratio) || !ratio_is_valid(error_correction_topk_ratio)) return 1;
    if (!method_is_valid(svd_uv_format) || !method_is_valid(svd_s_format) ||
        !method_is_valid(quantization_only_format))
        return 1;
    bitsqz_llm_decompress_release();
    const int rc = guarded([&] {
        decompress_init(g_decomp, num_rows, num_columns, outlier_topk_ratio, error_correction_topk_ratio, svd_ranks,
                        svd_uv_format, svd_s_format, quantization_only_format);
    });
    if (rc != 0) {
        const std::string msg = g_last_error;
        bitsqz_llm_decompress_release();
        set_error(msg.c_str());
    }
    return rc;
}

void bitsqz_llm_decompress_release() { g_decomp.release(); }

int bitsqz_llm_compress(const float *row_major_matrix_float_data, bitsqz_llm_array_t **out,
                        bitsqz_llm_compress_profile_t *profile) {
    if (!g_comp.initialized) return 1;
    if (!row_major_matrix_float_data || !out || *out) return 1;
    if (profile) *profile = bitsqz_llm_compress_profile_t{};
    return guarded([&] {
        Runtime &rt = g_comp;
        const uint64_t N = static_cast<uint64_t>(rt.rows) * rt.cols;
        const float *d_in = row_major_matrix_float_data;
        const hipEvent_t t_begin = rt.t_begin, t_end = rt.t_end;
        {
            if (profile) BSQ_HIP(hipEventRecord(t_begin, rt.stream));
            if (rt.input_location == BITSQZ_LLM_INPUT_HOST) {
                BSQ_HIP(hipMemcpyAsync(rt.d_stage, row_major_matrix_float_data, N * 4, hipMemcpyHostToDevice,
                                       rt.stream));
                d_in = rt.d_stage;
            }
            bsq_device_packed_t P{};
            compress_device(rt, d_in, &P, profile ? kAllEvents : kCopyEvents);
            // assemble_host returns once the copy stream has passed ev[6],
            // the end of the compute: nothing is left in flight
            bitsqz_llm_array_t *buf = assemble_host(rt, P);
            if (profile) {
                BSQ_HIP(hipEventRecord(t_end, rt.stream));
                BSQ_HIP(hipEventSynchronize(t_end));
                auto ms = [](hipEvent_t a, hipEvent_t b) {
                    float v = 0.0f;
                    return hipEventElapsedTime(&v, a, b) == hipSuccess ? static_cast<double>(v) : 0.0;
                };
                profile->topk_separation_latency_ms = ms(rt.ev[0], rt.ev[1]);
                profile->svd_lowrank_cuda_latency_ms = ms(rt.ev[1], rt.ev[2]);
                profile->quantization_compress_latency_ms = ms(rt.ev[2], rt.ev[3]);
                profile->reconsturct_quantization_decompress_latency_ms = ms(rt.ev[3], rt.ev[4]);
                profile->reconstruct_svd_latency_ms = ms(rt.ev[4], rt.ev[5]);
                profile->error_extraction_latency_ms = ms(rt.ev[5], rt.ev[6]);
                const double total = ms(t_begin, t_end);
                const double acc = profile->topk_separation_latency_ms + profile->svd_lowrank_cuda_latency_ms +
                                   profile->quantization_compress_latency_ms +
                                   profile->reconsturct_quantization_decompress_latency_ms +
                                   profile->reconstruct_svd_latency_ms + profile->error_extraction_latency_ms;
                profile->other_latency_ms = std::max(0.0, total - acc);
            }
            *out = buf;
        }
    });
}

int bitsqz_llm_decompress(const bitsqz_llm_array_t *compressed, float *d_dst, uint32_t dst_num_elements) {
    if (!g_decomp.initialized) return 1;
    if (!compressed || !d_dst || !compressed->payload) return 1;
    if (dst_num_elements < compressed->num_elements) return 1;
    if (!decompress_compatible(g_decomp, compressed)) return 1;
    return guarded([&] { decompress_host(g_decomp, compressed, d_dst); });
}

uint64_t bitsqz_llm_get_packed_size(const bitsqz_llm_array_t *c) {
    if (!c) return 0;
    const bitsqz_section_t secs[6] = {c->section_u, c->section_s, c->section_v, c->section_direct,
                                      c->section_outlier_topk, c->section_error_topk};
    uint64_t payload = 0;
    for (const auto &s : secs) {
        if (s.storage == BITSQZ_SECTION_NONE) continue;
        const uint64_t end = s.offset + s.size;
        if (end > payload) payload = end;
    }
    return static_cast<uint64_t>(sizeof(bitsqz_llm_array_t)) + payload;
}

// The payload end of the six sections without wrapping: false when 200 plus
// the largest end does not fit in 64 bits.  The reference sums in wrapping
// u64 arithmetic (src/bitsqz_llm.cu:1395-1415), so a header whose sections end
// within 200 bytes of 2^64 yields a packed size below 200, passes
// `buffer_size < packed_size` and is accepted with sections far outside the
// buffer; this build rejects it (the only difference from the reference's
// checks, and only for such headers).
static bool payload_end_fits(const bitsqz_llm_array_t *c, uint64_t buffer_size) {
    const bitsqz_section_t secs[6] = {c->section_u, c->section_s, c->section_v, c->section_direct,
                                      c->section_outlier_topk, c->section_error_topk};
    for (const auto &s : secs) {
        if (s.storage == BITSQZ_SECTION_NONE) continue;
        if (s.offset > UINT64_MAX - s.size) return false;
        if (s.offset + s.size > buffer_size - sizeof(bitsqz_llm_array_t)) return false;
    }
    return true;
}

bitsqz_llm_array_t *load_bitsqz_llm_from_buffer(const void *buffer, uint64_t buffer_size) {
    if (!buffer || buffer_size < sizeof(bitsqz_llm_array_t)) return nullptr;
    auto *c = static_cast<bitsqz_llm_array_t *>(std::calloc(1, static_cast<size_t>(buffer_size)));
    if (!c) return nullptr;
    std::memcpy(c, buffer, static_cast<size_t>(buffer_size));
    c->payload = reinterpret_cast<uint8_t *>(c) + sizeof(bitsqz_llm_array_t);
    const uint64_t packed = bitsqz_llm_get_packed_size(c);
    if (packed == 0 || buffer_size < packed || !payload_end_fits(c, buffer_size)) {
        std::free(c);
        return nullptr;
    }
    const uint64_t payload = packed - sizeof(bitsqz_llm_array_t);
    const bitsqz_section_t secs[6] = {c->section_u, c->section_s, c->section_v, c->section_direct,
                                      c->section_outlier_topk, c->section_error_topk};
    for (const auto &s : secs) {
        if (!section_bounds_ok(s, payload)) {
            std::free(c);
            return nullptr;
        }
    }
    return c;
}

void bitsqz_llm_free(bitsqz_llm_array_t *compressed) {
    if (!compressed) return;
    if (!BlockCache::get().put(compressed)) std::free(compressed);
}

// topk_compute_num_topk_columns: exported because the reference's ABI tests
// link it from topk_cuda_lib (tests/CMakeLists.txt:79-91,
// tests/bitsqz_llm/test_quantization.cpp:48).
__attribute__((visibility("default"))) uint16_t topk_compute_num_topk_columns(uint16_t num_columns,
                                                                             float topk_ratio) {
    return topk_num_columns(num_columns, topk_ratio);
}

// ===========================================================================
// extern "C" layer (include/bitsqz_llm_c.h)
// ===========================================================================
extern "C" {

const char *bsq_last_error(void) { return g_last_error.c_str(); }
const char *bsq_version(void) { return "bitsqz_llm-mi355x 0.1.0 (gfx950)"; }

int bsq_compress_initialize(uint16_t rows, uint16_t cols, float r_out, float r_err, int svd_ranks, int svd_niters,
                            int uv, int s, int direct, int loc) {
    return bitsqz_llm_compress_initialize(rows, cols, r_out, r_err, svd_ranks, svd_niters,
                                          static_cast<quantization_method_t>(uv),
                                          static_cast<quantization_method_t>(s),
                                          static_cast<quantization_method_t>(direct),
                                          static_cast<bitsqz_llm_input_location_t>(loc));
}
void bsq_compress_release(void) { bitsqz_llm_compress_release(); }
int bsq_decompress_initialize(uint16_t rows, uint16_t cols, float r_out, float r_err, int svd_ranks, int uv, int s,
                              int direct) {
    return bitsqz_llm_decompress_initialize(rows, cols, r_out, r_err, svd_ranks,
                                            static_cast<quantization_method_t>(uv),
                                            static_cast<quantization_method_t>(s),
                                            static_cast<quantization_method_t>(direct));
}
void bsq_decompress_release(void) { bitsqz_llm_decompress_release(); }
int bsq_compress(const float *in, bitsqz_llm_array_t **out, bitsqz_llm_compress_profile_t *profile) {
    return bitsqz_llm_compress(in, out, profile);
}
int bsq_decompress(const bitsqz_llm_array_t *c, float *d_dst, uint32_t n) { return bitsqz_llm_decompress(c, d_dst, n); }
uint64_t bsq_get_packed_size(const bitsqz_llm_array_t *c) { return bitsqz_llm_get_packed_size(c); }
bitsqz_llm_array_t *bsq_load_from_buffer(const void *b, uint64_t n) { return load_bitsqz_llm_from_buffer(b, n); }
void bsq_free(bitsqz_llm_array_t *c) { bitsqz_llm_free(c); }

int bsq_compress_set_sketch(const float *d_sketch) {
    if (!g_comp.initialized) {
        set_error("compress runtime not initialised");
        return 1;
    }
    g_comp.sketch = d_sketch;
    set_error("");
    return 0;
}

int bsq_device_compress(const float *d_input, bsq_device_packed_t *out) {
    if (!g_comp.initialized || !d_input || !out) {
        set_error("bsq_device_compress: runtime not initialised or null argument");
        return 1;
    }
    return guarded([&] { compress_device(g_comp, d_input, out, kNoEvents); });
}

int bsq_device_decompress(const bsq_device_packed_t *packed, float *d_dst, uint32_t dst_num_elements) {
    if (!g_decomp.initialized || !packed || !d_dst) {
        set_error("bsq_device_decompress: runtime not initialised or null argument");
        return 1;
    }
    return guarded([&] {
        const bitsqz_llm_array_t &H = packed->header;
        BSQ_REQUIRE(dst_num_elements >= H.num_elements, "destination too small");
        BSQ_REQUIRE(H.num_rows == g_decomp.rows && H.num_columns == g_decomp.cols, "shape mismatch");
        if (H.flags & kFlagSvd) {
            const uint16_t rank = static_cast<uint16_t>(H.effective_rank);
            BSQ_REQUIRE(rank != 0 && g_decomp.reconstruct_initialized && g_decomp.q == rank,
                        "rank mismatch with the decompress runtime");
        }
        const hipStream_t st = g_comp.initialized ? g_comp.stream : g_decomp.stream;
        // the error section is present iff the device flags word says so: the
        // scatter reads it on the device, so pass the full k and let the
        // kernel gate on the flag (no host synchronisation)
        decompress_device(g_decomp, *packed, packed->topk_k[1] > 0, d_dst, st, packed->d_flags);
    });
}

int bsq_device_synchronize(void) {
    return guarded([&] {
        if (g_comp.stream) BSQ_HIP(hipStreamSynchronize(g_comp.stream));
        if (g_decomp.stream) BSQ_HIP(hipStreamSynchronize(g_decomp.stream));
    });
}

void *bsq_runtime_stream(void) {
    return g_comp.initialized ? static_cast<void *>(g_comp.stream) : static_cast<void *>(g_decomp.stream);
}

// ---------------------------------------------------------------------------
// Lanes: independent compress + decompress runtime pairs, each on its own
// non-blocking stream (default priority), for callers with several matrices
// in flight.  A lane's round trip is the device-resident pipeline of
// bsq_device_compress + bsq_device_decompress on its own buffers, so lanes
// share nothing and need no ordering between them; the one-CU stages of one
// lane's randomised SVD then run beside the other lanes' matrix-core GEMMs.
// ---------------------------------------------------------------------------
namespace {
struct Lane {
    Runtime comp, decomp;
    bsq_device_packed_t last{};
};
std::vector<std::unique_ptr<Lane>> g_lanes;

void lanes_release() noexcept {
    for (auto &l : g_lanes) {
        l->decomp.release();
        l->comp.release();
    }
    g_lanes.clear();
}
}  // namespace

int bsq_lanes_initialize(int lanes, uint16_t rows, uint16_t cols, float r_out, float r_err, int svd_ranks,
                         int svd_niters, int uv, int s, int direct) {
    lanes_release();
    if (lanes < 1 || lanes > 8 || rows == 0 || cols == 0 || svd_niters < 1) {
        set_error("bsq_lanes_initialize: 1 to 8 lanes, a non-empty shape and svd_niters >= 1");
        return 1;
    }
    if (!ratio_is_valid(r_out) || !ratio_is_valid(r_err) || !method_is_valid(uv) || !method_is_valid(s) ||
        !method_is_valid(direct)) {
        set_error("bsq_lanes_initialize: invalid ratio or method");
        return 1;
    }
    const int rc = guarded([&] {
        const int q = svd_ranks >= 1 ? std::max(1, std::min(svd_ranks, static_cast<int>(std::min(rows, cols)))) : -1;
        for (int i = 0; i < lanes; ++i) {
            auto l = std::make_unique<Lane>();
            // one stream per lane (a process has few hardware queues: with
            // GPU_MAX_HW_QUEUES at its default of 4, extra streams share them
            // and their work serialises), no copy stream, no host staging
            compress_init(l->comp, rows, cols, r_out, r_err, svd_ranks, svd_niters, uv, s, direct,
                          BITSQZ_LLM_INPUT_DEVICE, false);
            decompress_init(l->decomp, rows, cols, r_out, r_err, q, uv, s, direct, l->comp.stream);
            g_lanes.push_back(std::move(l));
        }
    });
    if (rc != 0) {
        const std::string msg = g_last_error;
        lanes_release();
        set_error(msg.c_str());
    }
    return rc;
}

int bsq_lanes_roundtrip(int lane, const float *d_input, float *d_dst) {
    if (lane < 0 || lane >= static_cast<int>(g_lanes.size()) || !d_input || !d_dst) {
        set_error("bsq_lanes_roundtrip: no such lane or null pointer");
        return 1;
    }
    return guarded([&] {
        Lane &l = *g_lanes[lane];
        compress_device(l.comp, d_input, &l.last, kNoEvents);
        decompress_device(l.decomp, l.last, l.last.topk_k[1] > 0, d_dst, l.comp.stream, l.last.d_flags);
    });
}

void *bsq_lanes_stream(int lane) {
    if (lane < 0 || lane >= static_cast<int>(g_lanes.size())) return nullptr;
    return g_lanes[lane]->comp.stream;
}

int bsq_lanes_synchronize(void) {
    return guarded([&] {
        for (auto &l : g_lanes) BSQ_HIP(hipStreamSynchronize(l->comp.stream));
    });
}

void bsq_lanes_release(void) { lanes_release(); }

int bsq_topk_num_columns(uint16_t num_columns, float ratio, uint16_t *out_k) {
    return guarded([&] {
        BSQ_REQUIRE(out_k != nullptr, "null output");
        *out_k = topk_num_columns(num_columns, ratio);
    });
}

int bsq_topk_select(const float *d_input, uint16_t rows, uint16_t cols, uint16_t k, uint16_t *d_indices,
                    float *d_values, float *d_residual, void *stream) {
    return guarded([&] {
        TopkArgs a;
        a.a = d_input;
        a.rows = rows;
        a.cols = cols;
        a.k = k;
        a.indices = d_indices;
        a.values = d_values;
        a.residual = d_residual;
        launch_topk_select(a, static_cast<hipStream_t>(stream));
    });
}

int bsq_topk_scatter(const uint16_t *d_indices, const float *d_values, uint16_t rows, uint16_t cols, uint16_t k,
                     float *d_dense, int accumulate, void *stream) {
    return guarded([&] {
        launch_topk_scatter(d_indices, d_values, k, nullptr, nullptr, 0, rows, cols, d_dense, accumulate != 0,
                            static_cast<hipStream_t>(stream));
    });
}

int bsq_quant_compress(const float *d_input, uint64_t count, int method, float *d_scales_f32, uint8_t *d_scales_u8,
                       float *d_dq_scale, uint8_t *d_codes, void *stream) {
    return guarded([&] {
        static uint32_t *scratch = nullptr;
        if (method == kMethodNF4DQ && scratch == nullptr) scratch = dev_alloc<uint32_t>(1);
        launch_quant_encode(d_input, count, method, d_scales_f32, d_scales_u8, d_dq_scale, d_codes, scratch,
                            static_cast<hipStream_t>(stream));
    });
}

int bsq_quant_decompress(uint64_t count, int method, const float *d_scales_f32, const uint8_t *d_scales_u8,
                         const float *d_dq_scale, const uint8_t *d_codes, float *d_output, void *stream) {
    return guarded([&] {
        launch_quant_decode(count, method, d_scales_f32, d_scales_u8, d_dq_scale, d_codes, d_output,
                            static_cast<hipStream_t>(stream));
    });
}

int bsq_quant_nf4_codes(const float *d_values, uint64_t n, uint8_t *d_codes, void *stream) {
    return guarded([&] { launch_nf4_code_batch(d_values, n, d_codes, static_cast<hipStream_t>(stream)); });
}
int bsq_quant_e4m3_encode(const float *d_values, uint64_t n, uint8_t *d_codes, void *stream) {
    return guarded([&] { launch_e4m3_encode_batch(d_values, n, d_codes, static_cast<hipStream_t>(stream)); });
}
int bsq_quant_e4m3_decode(const uint8_t *d_codes, uint64_t n, float *d_values, void *stream) {
    return guarded([&] { launch_e4m3_decode_batch(d_codes, n, d_values, static_cast<hipStream_t>(stream)); });
}
int bsq_quant_nf4_code_sweep(uint64_t lo, uint64_t hi, unsigned long long *d_hist16, unsigned long long *d_checksum,
                             void *stream) {
    return guarded(
        [&] { launch_nf4_code_sweep(lo, hi, d_hist16, d_checksum, static_cast<hipStream_t>(stream)); });
}
void bsq_nf4_thresholds(float out[15]) {
    const float t[15] = BSQ_NF4_THRESHOLDS;
    for (int i = 0; i < 15; ++i) out[i] = t[i];
}

int bsq_svd_lowrank(const float *d_A, int m, int n, int q, int niter, const float *d_sketch, uint64_t seed,
                    float *d_U, float *d_S, float *d_V, void *stream) {
    return guarded([&] {
        BSQ_REQUIRE(m > 0 && n > 0 && q > 0 && niter >= 0, "svd: bad shape");
        SvdPlan *plan = svd_plan_create(m, n, q, niter);
        try {
            svd_run(plan, d_A, d_sketch, seed, d_U, d_S, d_V, static_cast<hipStream_t>(stream));
            BSQ_HIP(hipStreamSynchronize(static_cast<hipStream_t>(stream)));
        } catch (...) {
            svd_plan_destroy(plan);
            throw;
        }
        svd_plan_destroy(plan);
    });
}

int bsq_svd_lowrank_noalloc(const float *d_A, int m, int n, int q, int niter, const float *d_sketch, uint64_t seed,
                            float *d_U, float *d_S, float *d_V, void *stream) {
    return guarded([&] {
        svd_run_noalloc(d_A, m, n, q, niter, d_sketch, seed, d_U, d_S, d_V, static_cast<hipStream_t>(stream));
    });
}

int bsq_reconstruct_lowrank(const float *d_U, const float *d_S, const float *d_V, int m, int n, int k, float *d_out,
                            void *stream) {
    return guarded([&] {
        BSQ_REQUIRE(m > 0 && n > 0 && k > 0, "reconstruct: bad shape");
        launch_reconstruct(d_U, d_S, d_V, m, n, k, nullptr, d_out, static_cast<hipStream_t>(stream));
    });
}

int bsq_gaussian_fill(float *d_out, uint64_t n, uint64_t seed, void *stream) {
    return guarded([&] { launch_gaussian_fill(d_out, n, seed, static_cast<hipStream_t>(stream)); });
}

// device memory helpers for FFI callers without a GPU framework
int bsq_device_malloc(void **ptr, uint64_t bytes) { return guarded([&] { BSQ_HIP(hipMalloc(ptr, bytes)); }); }
int bsq_device_free(void *ptr) { return guarded([&] { BSQ_HIP(hipFree(ptr)); }); }
int bsq_memcpy_h2d(void *dst, const void *src, uint64_t bytes) {
    return guarded([&] { BSQ_HIP(hipMemcpy(dst, src, bytes, hipMemcpyHostToDevice)); });
}
int bsq_memcpy_d2h(void *dst, const void *src, uint64_t bytes) {
    return guarded([&] { BSQ_HIP(hipMemcpy(dst, src, bytes, hipMemcpyDeviceToHost)); });
}
int bsq_memcpy_d2d(void *dst, const void *src, uint64_t bytes) {
    return guarded([&] { BSQ_HIP(hipMemcpy(dst, src, bytes, hipMemcpyDeviceToDevice)); });
}
int bsq_device_memset(void *dst, int value, uint64_t bytes) {
    return guarded([&] { BSQ_HIP(hipMemset(dst, value, bytes)); });
}
int bsq_host_malloc(void **ptr, uint64_t bytes) {
    return guarded([&] { BSQ_HIP(hipHostMalloc(ptr, bytes, hipHostMallocDefault)); });
}
int bsq_host_free(void *ptr) { return guarded([&] { BSQ_HIP(hipHostFree(ptr)); }); }
int bsq_memcpy_h2d_async(void *dst, const void *src, uint64_t bytes, void *stream) {
    return guarded(
        [&] { BSQ_HIP(hipMemcpyAsync(dst, src, bytes, hipMemcpyHostToDevice, static_cast<hipStream_t>(stream))); });
}
int bsq_stream_synchronize(void *stream) {
    return guarded([&] { BSQ_HIP(hipStreamSynchronize(static_cast<hipStream_t>(stream))); });
}
int bsq_device_count(int *count) { return guarded([&] { BSQ_HIP(hipGetDeviceCount(count)); }); }
int bsq_event_create(void **event) {
    return guarded([&] {
        hipEvent_t e = nullptr;
        BSQ_HIP(hipEventCreate(&e));
        *event = e;
    });
}
int bsq_event_destroy(void *event) {
    return guarded([&] { BSQ_HIP(hipEventDestroy(static_cast<hipEvent_t>(event))); });
}
int bsq_event_record(void *event, void *stream) {
    return guarded(
        [&] { BSQ_HIP(hipEventRecord(static_cast<hipEvent_t>(event), static_cast<hipStream_t>(stream))); });
}
int bsq_copy_kernel(const void *d_src, void *d_dst, uint64_t bytes, void *stream) {
    return guarded([&] {
        BSQ_REQUIRE(d_src && d_dst && bytes % 16 == 0, "copy kernel: null pointer or size not a multiple of 16");
        BSQ_REQUIRE((reinterpret_cast<uintptr_t>(d_src) | reinterpret_cast<uintptr_t>(d_dst)) % 16 == 0,
                    "copy kernel: pointers must be 16-byte aligned");
        const uint64_t n4 = bytes / 16;
        if (n4 == 0) return;
        uint64_t grid = ceil_div(n4, 256);
        const uint64_t cap = static_cast<uint64_t>(cu_count()) * 16;
        if (grid > cap) grid = cap;
        copy_f32x4_kernel<<<static_cast<unsigned>(grid), 256, 0, static_cast<hipStream_t>(stream)>>>(
            static_cast<const float4 *>(d_src), static_cast<float4 *>(d_dst), n4);
        BSQ_HIP(hipGetLastError());
    });
}

int bsq_kernel_timer_start(void) {
    return guarded([&] {
        g_timer_on = true;
        for (auto &t : g_gemm_timer) t.used = 0;
    });
}

int bsq_kernel_timer_stop(double *total_ms, int *launches) {
    return guarded([&] {
        BSQ_REQUIRE(total_ms && launches, "null output");
        g_timer_on = false;
        for (auto &t : g_gemm_timer) t.read();
        *total_ms = g_gemm_timer[kTimeReconstruct].last_ms;
        *launches = g_gemm_timer[kTimeReconstruct].last_launches;
    });
}

int bsq_kernel_timer_read(int timer_class, double *total_ms, int *launches) {
    return guarded([&] {
        BSQ_REQUIRE(total_ms && launches, "null output");
        BSQ_REQUIRE(timer_class >= 0 && timer_class < kTimeClasses, "unknown timer class");
        *total_ms = g_gemm_timer[timer_class].last_ms;
        *launches = g_gemm_timer[timer_class].last_launches;
    });
}

int bsq_event_elapsed_ms(void *start, void *stop, float *ms) {
    return guarded([&] {
        BSQ_HIP(hipEventSynchronize(static_cast<hipEvent_t>(stop)));
        BSQ_HIP(hipEventElapsedTime(ms, static_cast<hipEvent_t>(start), static_cast<hipEvent_t>(stop)));
    });
}

}  // extern "C"
