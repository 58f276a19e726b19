// stream_check: the weight streamer's host side and the C ABI's argument
// checks, run from a host build under AddressSanitizer and UBSan
// (`make asan` in this directory; the GPU code is the ordinary build).
//
// - A ring of 4 slots streams 11 layers of 3 MiB + 123 bytes (not a multiple
//   of the 4 KiB slot granule) from pinned host memory, two loads ahead, with
//   copy timing on; every slot is read back and compared with its layer.
// - The copy log: a count query, a partial read that keeps the log, a full
//   read that clears it, an empty read after that.
// - Refusals: loading into a slot that was loaded and not released, slot ids
//   out of range, a copy larger than a slot, a third copy stream, a streamer
//   of no slots; then destroying a streamer whose copies are still pending.
// - Argument checks of df_absmax_f32 and df_fp8_gemm_fwd (NULL operands, a
//   negative size): refused before any launch.
#include <hip/hip_runtime.h>

#include <cstdio>
#include <cstring>
#include <vector>

#include "df_capi.h"

#define REQUIRE(c)                                                                                   \
    do {                                                                                             \
        if (!(c)) {                                                                                  \
            std::printf("FAIL %s:%d %s | %s\n", __FILE__, __LINE__, #c, df_last_error_string());      \
            return 1;                                                                                \
        }                                                                                            \
    } while (0)

int main() {
    hipStream_t st;
    REQUIRE(hipStreamCreate(&st) == hipSuccess);
    const size_t bytes = (3u << 20) + 123;
    const int layers = 11, slots = 4, ahead = slots - 2;
    void* host = nullptr;
    REQUIRE(df_host_alloc(bytes * layers, &host) == DF_OK);
    unsigned char* h = static_cast<unsigned char*>(host);
    for (size_t i = 0; i < bytes * layers; ++i) h[i] = (unsigned char)(i * 131 + 7);

    df_streamer* s = nullptr;
    REQUIRE(df_streamer_create(0, bytes, &s) != DF_OK && s == nullptr);
    REQUIRE(df_streamer_create(slots, bytes, nullptr) != DF_OK);
    REQUIRE(df_streamer_create(slots, bytes, &s) == DF_OK && s);
    REQUIRE(df_streamer_set_timing(s, 1) == DF_OK);
    void* cs = nullptr;
    REQUIRE(df_streamer_copy_stream(s, 0, &cs) == DF_OK && cs);
    REQUIRE(df_streamer_copy_stream(s, 1, &cs) == DF_OK && cs);
    REQUIRE(df_streamer_copy_stream(s, 2, &cs) != DF_OK);

    std::vector<int> slot(layers);
    std::vector<void*> dev(layers);
    std::vector<unsigned char> back(bytes);
    for (int l = 0; l < ahead; ++l) REQUIRE(df_streamer_load(s, h + l * bytes, bytes, &slot[l], &dev[l]) == DF_OK);
    for (int l = 0; l < layers; ++l) {
        REQUIRE(df_streamer_wait(s, slot[l], st) == DF_OK);
        REQUIRE(hipMemcpyAsync(back.data(), dev[l], bytes, hipMemcpyDeviceToHost, st) == hipSuccess);
        REQUIRE(hipStreamSynchronize(st) == hipSuccess);
        REQUIRE(std::memcmp(back.data(), h + l * bytes, bytes) == 0);
        REQUIRE(df_streamer_release(s, slot[l], st) == DF_OK);
        if (l + ahead < layers)
            REQUIRE(df_streamer_load(s, h + (l + ahead) * bytes, bytes, &slot[l + ahead], &dev[l + ahead]) == DF_OK);
    }

    int n = -1;
    std::vector<float> t0(layers), t1(layers);
    REQUIRE(df_streamer_copy_log(s, nullptr, nullptr, 0, &n) == DF_OK && n == layers);
    REQUIRE(df_streamer_copy_log(s, t0.data(), t1.data(), 3, &n) == DF_OK && n == layers);
    REQUIRE(df_streamer_copy_log(s, t0.data(), t1.data(), layers, &n) == DF_OK && n == layers);
    for (int i = 0; i < layers; ++i) REQUIRE(t0[i] >= 0.f && t1[i] >= t0[i]);
    REQUIRE(df_streamer_copy_log(s, t0.data(), t1.data(), layers, &n) == DF_OK && n == 0);

    int k;
    void* d;
    for (int i = 0; i < slots; ++i) REQUIRE(df_streamer_load(s, host, bytes, &k, &d) == DF_OK);
    REQUIRE(df_streamer_load(s, host, bytes, &k, &d) == DF_ERR_INVALID);
    REQUIRE(df_streamer_wait(s, slots, st) != DF_OK);
    REQUIRE(df_streamer_release(s, -1, st) != DF_OK);
    REQUIRE(df_streamer_slot(s, slots, &d) != DF_OK);
    REQUIRE(df_streamer_load(s, host, bytes + 2 * 4096, &k, &d) != DF_OK);
    REQUIRE(df_streamer_destroy(s) == DF_OK);
    REQUIRE(df_host_free(host) == DF_OK);

    float* f = nullptr;
    REQUIRE(hipMalloc(&f, 1 << 20) == hipSuccess);
    REQUIRE(df_absmax_f32(nullptr, 16, f, f + 16, 4096, st) != DF_OK);
    REQUIRE(df_absmax_f32(f, -1, f + 8, f + 16, 4096, st) != DF_OK);
    REQUIRE(df_fp8_gemm_fwd(nullptr, 16, nullptr, 16, 4, 4, 16, f, f, DF_DTYPE_FLOAT32, nullptr, DF_DTYPE_FLOAT32, f,
                            4, nullptr, 0, st) != DF_OK);
    REQUIRE(hipStreamSynchronize(st) == hipSuccess);
    REQUIRE(hipFree(f) == hipSuccess);
    REQUIRE(hipStreamDestroy(st) == hipSuccess);
    std::printf("stream_check: all checks passed\n");
    return 0;
}
