// Downstream caller of the nine C++-linkage functions of bitsqz_llm.hpp,
// linked through the installed CMake package.  Two scenarios, each writing
// the packed object and the decoded matrix to <outdir> for the Python test
// to check against the oracle:
//   walk:   the 8 x 8 host-input case of the reference's walkthrough
//           (examples/bitsqz_llm_walkthrough.cpp:34-121): rank 4, two power
//           iterations, NF4 U/V and S, through the inline two-argument
//           bitsqz_llm_compress overload; the object is copied to a byte
//           buffer and reloaded with load_bitsqz_llm_from_buffer first;
//   direct: 64 x 512 device input, NF4_DQ direct section with outlier and
//           error top-k, through the three-argument form with a profile.
// It also checks the contract's failure returns.  Exit code 0 = all good.
#include <bitsqz_llm.hpp>

#include <hip/hip_runtime.h>

#include <cmath>
#include <cstdio>
#include <cstring>
#include <string>
#include <vector>

#define CHECK(cond, what)                                   \
    do {                                                    \
        if (!(cond)) {                                      \
            std::fprintf(stderr, "consumer: %s\n", what);   \
            return 1;                                       \
        }                                                   \
    } while (0)

static bool write_file(const std::string &path, const void *data, size_t n) {
    FILE *f = std::fopen(path.c_str(), "wb");
    if (!f) return false;
    const bool ok = std::fwrite(data, 1, n, f) == n;
    return std::fclose(f) == 0 && ok;
}

static int walkthrough(const std::string &dir) {
    constexpr uint16_t rows = 8, cols = 8;
    std::vector<float> x(rows * cols);
    for (size_t i = 0; i < x.size(); ++i) x[i] = static_cast<float>((i % cols) * 0.25f + (i / cols) * 0.5f);
    CHECK(bitsqz_llm_compress_initialize(rows, cols, 0.0f, 0.0f, 4, 2, NF4, NF4, quantization_NONE,
                                         BITSQZ_LLM_INPUT_HOST) == 0, "compress_initialize (walk)");
    CHECK(bitsqz_llm_decompress_initialize(rows, cols, 0.0f, 0.0f, 4, NF4, NF4, quantization_NONE) == 0,
          "decompress_initialize (walk)");
    bitsqz_llm_array_t *packed = nullptr;
    CHECK(bitsqz_llm_compress(x.data(), &packed) == 0 && packed, "compress (two-argument overload)");
    bitsqz_llm_array_t *again = packed;
    CHECK(bitsqz_llm_compress(x.data(), &again) == 1, "compress must refuse a non-null *out");
    const uint64_t size = bitsqz_llm_get_packed_size(packed);
    CHECK(size > sizeof(bitsqz_llm_array_t), "packed size");
    std::vector<unsigned char> bytes(size);
    std::memcpy(bytes.data(), packed, size);
    bitsqz_llm_free(packed);
    CHECK(load_bitsqz_llm_from_buffer(bytes.data(), size - 1) == nullptr, "truncated buffer must not load");
    bitsqz_llm_array_t *loaded = load_bitsqz_llm_from_buffer(bytes.data(), size);
    CHECK(loaded != nullptr && loaded->payload == reinterpret_cast<unsigned char *>(loaded) + 200, "reload");
    float *d_out = nullptr;
    CHECK(hipMalloc(&d_out, x.size() * sizeof(float)) == hipSuccess, "hipMalloc");
    CHECK(bitsqz_llm_decompress(loaded, d_out, rows * cols - 1) == 1, "short destination must be refused");
    CHECK(bitsqz_llm_decompress(loaded, d_out, rows * cols) == 0, "decompress (walk)");
    std::vector<float> y(x.size());
    CHECK(hipMemcpy(y.data(), d_out, y.size() * 4, hipMemcpyDeviceToHost) == hipSuccess, "hipMemcpy");
    double mae = 0.0;
    for (size_t i = 0; i < x.size(); ++i) mae += std::fabs(static_cast<double>(x[i]) - y[i]);
    std::printf("walk: packed %llu bytes, mean absolute error %.6f\n", static_cast<unsigned long long>(size),
                mae / x.size());
    CHECK(write_file(dir + "/walk_packed.bin", bytes.data(), size), "write walk_packed.bin");
    CHECK(write_file(dir + "/walk_decoded.bin", y.data(), y.size() * 4), "write walk_decoded.bin");
    bitsqz_llm_free(loaded);
    (void)hipFree(d_out);
    bitsqz_llm_compress_release();
    bitsqz_llm_decompress_release();
    bitsqz_llm_array_t *none = nullptr;
    CHECK(bitsqz_llm_compress(x.data(), &none) == 1, "compress after release must fail");
    return 0;
}

static int direct(const std::string &dir) {
    constexpr uint16_t rows = 64, cols = 512;
    std::vector<float> x(rows * cols);
    uint32_t s = 12345u;
    for (size_t i = 0; i < x.size(); ++i) {  // xorshift values in [-4, 4), column 7 scaled as an outlier channel
        s ^= s << 13;
        s ^= s >> 17;
        s ^= s << 5;
        x[i] = (static_cast<float>(s >> 8) / 16777216.0f - 0.5f) * 8.0f * ((i % cols) == 7 ? 50.0f : 1.0f);
    }
    float *d_in = nullptr, *d_out = nullptr;
    CHECK(hipMalloc(&d_in, x.size() * 4) == hipSuccess && hipMalloc(&d_out, x.size() * 4) == hipSuccess, "hipMalloc");
    CHECK(hipMemcpy(d_in, x.data(), x.size() * 4, hipMemcpyHostToDevice) == hipSuccess, "hipMemcpy");
    CHECK(bitsqz_llm_compress_initialize(rows, cols, 0.01f, 0.02f, -1, 1, quantization_NONE, quantization_NONE,
                                         NF4_DQ, BITSQZ_LLM_INPUT_DEVICE) == 0, "compress_initialize (direct)");
    CHECK(bitsqz_llm_decompress_initialize(rows, cols, 0.01f, 0.02f, -1, quantization_NONE, quantization_NONE,
                                           NF4_DQ) == 0, "decompress_initialize (direct)");
    bitsqz_llm_compress_profile_t prof{};
    bitsqz_llm_array_t *packed = nullptr;
    CHECK(bitsqz_llm_compress(d_in, &packed, &prof) == 0 && packed, "compress (with profile)");
    CHECK(prof.topk_separation_latency_ms >= 0.0 && prof.other_latency_ms >= 0.0, "profile");
    const uint64_t size = bitsqz_llm_get_packed_size(packed);
    CHECK(bitsqz_llm_decompress(packed, d_out, rows * cols) == 0, "decompress (direct)");
    std::vector<float> y(x.size());
    CHECK(hipMemcpy(y.data(), d_out, y.size() * 4, hipMemcpyDeviceToHost) == hipSuccess, "hipMemcpy");
    std::printf("direct: packed %llu bytes, flags %u\n", static_cast<unsigned long long>(size), packed->flags);
    CHECK(write_file(dir + "/direct_input.bin", x.data(), x.size() * 4), "write direct_input.bin");
    CHECK(write_file(dir + "/direct_packed.bin", packed, size), "write direct_packed.bin");
    CHECK(write_file(dir + "/direct_decoded.bin", y.data(), y.size() * 4), "write direct_decoded.bin");
    bitsqz_llm_free(packed);
    // the runtimes are independent: the decompressor outlives the compressor
    bitsqz_llm_compress_release();
    CHECK(bitsqz_llm_get_packed_size(nullptr) == 0, "get_packed_size(nullptr)");
    bitsqz_llm_decompress_release();
    (void)hipFree(d_in);
    (void)hipFree(d_out);
    return 0;
}

int main(int argc, char **argv) {
    const std::string dir = argc > 1 ? argv[1] : ".";
    if (walkthrough(dir) != 0) return 1;
    if (direct(dir) != 0) return 1;
    std::printf("consumer: ok\n");
    return 0;
}
