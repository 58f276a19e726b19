// C++ drop-in tests (namespace dnn), shaped like the reference's GTest
// suites: tests/core/cuda_test.cu (-> HipTest), tests/core/tensor_test.cu
// (-> TensorTest), tests/layers/fully_connected_layer_test.cu
// (-> FullyConnectedLayerTest), tests/optimizers/adam_optimizer_test.cu
// (-> AdamOptimizerTest), plus the fp8 tensor conversions and gradient
// clipping (-> ClipGradNormTest).
//
// Expected values of the fp8 path come from the CPU oracle
// (oracle/libdf_oracle.so): the operands are quantized and dequantized by
// the oracle and the reference's fp32 loops run on them.  Where the
// reference's test checks the fp32 product to 1e-5, these tests check the
// fp8 product to the same 1e-5 and the fp32 product to the fp8 error bound.
#include <hip/hip_runtime.h>

#include <algorithm>
#include <cmath>
#include <cstring>
#include <memory>
#include <random>
#include <sstream>
#include <thread>
#include <vector>

#include "df_oracle.h"
#include "dnn/core/hip.hpp"
#include "dnn/core/tensor.hpp"
#include "dnn/layers/fully_connected_layer.hpp"
#include "dnn/layers/layer_norm_layer.hpp"
#include "dnn/optimizers/adam_optimizer.hpp"
#include "dnn/utils/common.hpp"
#include "mini_test.hpp"

using namespace dnn;

namespace {

std::vector<float> uniform(size_t n, float lo, float hi, unsigned seed) {
    std::mt19937 g(seed);
    std::uniform_real_distribution<float> d(lo, hi);
    std::vector<float> v(n);
    for (auto& x : v) x = d(g);
    return v;
}

// oracle: per-tensor absmax quantize then dequantize (the values the GEMM sees)
std::vector<float> fp8_values(const std::vector<float>& x, int fmt) {
    const int64_t n = (int64_t)x.size();
    const float s = dfo_scale(dfo_absmax_f32(x.data(), n), fmt);
    std::vector<uint8_t> q(n);
    std::vector<float> d(n);
    dfo_quantize_f32(x.data(), n, s, fmt, q.data());
    dfo_dequantize_f32(q.data(), n, s, fmt, d.data());
    return d;
}

std::vector<float> bf16_to_float(const std::vector<uint16_t>& h) {
    std::vector<float> f(h.size());
    for (size_t i = 0; i < h.size(); ++i) f[i] = dfo_bf16_to_f32(h[i]);
    return f;
}

std::vector<uint16_t> float_to_bf16(const std::vector<float>& f) {
    std::vector<uint16_t> h(f.size());
    for (size_t i = 0; i < f.size(); ++i) h[i] = dfo_f32_to_bf16(f[i]);
    return h;
}

// max|y - r| / max|r|: the normwise relative error of the fp8 GEMM contract
double rel_err(const std::vector<float>& y, const std::vector<float>& r) {
    double num = 0, den = 0;
    for (size_t i = 0; i < r.size(); ++i) {
        num = std::max(num, (double)std::fabs(y[i] - r[i]));
        den = std::max(den, (double)std::fabs(r[i]));
    }
    return den > 0 ? num / den : num;
}

template <typename TT>
std::vector<TT> download(const tensor<TT>& t) {
    std::vector<TT> h(t.size());
    t.download(h.data());
    return h;
}

std::vector<float> download_f(const tensor<bfloat16>& t) {
    std::vector<uint16_t> h(t.size());
    t.download(reinterpret_cast<bfloat16*>(h.data()));
    return bf16_to_float(h);
}

void upload_bf16(tensor<bfloat16>& t, const std::vector<float>& v) {
    const auto h = float_to_bf16(v);
    t.upload(reinterpret_cast<const bfloat16*>(h.data()));
}

// binary16 through the oracle's conversions (dfo_f32_to_f16: nearest even)
std::vector<float> round_f16(const std::vector<float>& f) {
    std::vector<float> r(f.size());
    for (size_t i = 0; i < f.size(); ++i) r[i] = dfo_f16_to_f32(dfo_f32_to_f16(f[i]));
    return r;
}

std::vector<float> download_f(const tensor<__half>& t) {
    std::vector<uint16_t> h(t.size());
    t.download(reinterpret_cast<__half*>(h.data()));
    std::vector<float> f(h.size());
    for (size_t i = 0; i < h.size(); ++i) f[i] = dfo_f16_to_f32(h[i]);
    return f;
}

void upload_f16(tensor<__half>& t, const std::vector<float>& v) {
    std::vector<uint16_t> h(v.size());
    for (size_t i = 0; i < v.size(); ++i) h[i] = dfo_f32_to_f16(v[i]);
    t.upload(reinterpret_cast<const __half*>(h.data()));
}

class HipFixture : public mini_test::Test {
protected:
    std::unique_ptr<Hip> hip_;
    void SetUp() override {
        hip_ = std::make_unique<Hip>(0);
        (void)hipDeviceSynchronize();
    }
    void TearDown() override {
        (void)hipDeviceSynchronize();
        hip_.reset();
        Hip::set_stream(nullptr);
    }
};

using HipTest = HipFixture;
using TensorTest = HipFixture;
using Fp8TensorTest = HipFixture;
using FullyConnectedLayerTest = HipFixture;
using AdamOptimizerTest = HipFixture;
using LayerNormLayerTest = HipFixture;
using ClipGradNormTest = HipFixture;

}  // namespace

// ============================================================== HipTest ==
TEST_F(HipTest, Constructor) {
    EXPECT_NO_THROW({
        Hip hip;
        EXPECT_EQ(hip.id(), 0);
    });
    int device_count = 0;
    (void)hipGetDeviceCount(&device_count);
    EXPECT_THROW(Hip hip(device_count), std::runtime_error);
    (void)hipSetDevice(0);
}

TEST_F(HipTest, CurrentInstance) {
    hip_.reset();
    {
        Hip h1(0);
        EXPECT_EQ(&Hip::current(), &h1);
        {
            Hip h2(0);
            EXPECT_EQ(&Hip::current(), &h2);
        }
    }
    EXPECT_THROW(Hip::current(), std::runtime_error);
}

TEST_F(HipTest, GetDevices) {
    const auto& devices = Hip::get_devices();
    int device_count = 0;
    (void)hipGetDeviceCount(&device_count);
    EXPECT_EQ((int)devices.size(), device_count);
    for (size_t i = 0; i < devices.size(); ++i) {
        EXPECT_EQ(devices[i].id(), (int)i);
        EXPECT_FALSE(devices[i].name().empty());
        EXPECT_EQ(devices[i].architecture_name().rfind("gfx950", 0), 0u);
        EXPECT_GT(devices[i].num_sm(), 0);
        EXPECT_GT(devices[i].available_memory_bytes(), 0u);
    }
}

TEST_F(HipTest, DumpInfo) {
    Hip hip;
    std::stringstream ss;
    hip.dump_info(ss);
    const std::string info = ss.str();
    EXPECT_TRUE(info.find("[HIP System Summary]") != std::string::npos);
    EXPECT_TRUE(info.find("HIP Device") != std::string::npos);
}

TEST_F(HipTest, ThreadSafety) {
    Hip* seen[2] = {nullptr, nullptr};
    std::thread t1([&] {
        Hip h(0);
        seen[0] = &Hip::current();
    });
    std::thread t2([&] {
        Hip h(0);
        seen[1] = &Hip::current();
    });
    t1.join();
    t2.join();
    EXPECT_NE(seen[0], nullptr);
    EXPECT_NE(seen[1], nullptr);
    EXPECT_EQ(&Hip::current(), hip_.get());  // other threads leave ours alone
}

TEST_F(HipTest, DefaultStreamIsLegacy) { EXPECT_EQ(Hip::stream(), hipStreamLegacy); }

TEST_F(HipTest, SetAndGetStream) {
    hipStream_t s;
    ASSERT_EQ(hipStreamCreate(&s), hipSuccess);
    Hip::set_stream(s);
    EXPECT_EQ(Hip::stream(), s);
    Hip::set_stream(nullptr);
    EXPECT_EQ(Hip::stream(), hipStreamLegacy);
    (void)hipStreamDestroy(s);
}

TEST_F(HipTest, StreamGuardRestoresPreviousStream) {
    hipStream_t s1, s2;
    ASSERT_EQ(hipStreamCreate(&s1), hipSuccess);
    ASSERT_EQ(hipStreamCreate(&s2), hipSuccess);
    Hip::set_stream(s1);
    EXPECT_EQ(Hip::stream(), s1);
    {
        StreamGuard guard(s2);
        EXPECT_EQ(Hip::stream(), s2);
    }
    EXPECT_EQ(Hip::stream(), s1);
    Hip::set_stream(nullptr);
    (void)hipStreamDestroy(s1);
    (void)hipStreamDestroy(s2);
}

// =========================================================== TensorTest ==
TEST_F(TensorTest, ConstructorAndShape) {
    std::vector<int> shape = {2, 3, 4};
    tensor<float> t(shape);
    EXPECT_TRUE(t.shape() == shape);
    EXPECT_EQ(t.size(), 24);
    EXPECT_EQ(t.size(0), 2);
    EXPECT_EQ(t.size(1), 3);
    EXPECT_EQ(t.size(2), 4);
    EXPECT_THROW(t.size(3), std::out_of_range);
}

TEST_F(TensorTest, UploadDownload) {
    tensor<float> t({2, 2});
    std::vector<float> host = {1.0f, 2.0f, 3.0f, 4.0f};
    t.upload(host.data());
    const auto back = download(t);
    for (size_t i = 0; i < host.size(); ++i) EXPECT_FLOAT_EQ(host[i], back[i]);
}

TEST_F(TensorTest, FillAndZero) {
    tensor<float> t({2, 2});
    t.fill(1.0f);
    for (float v : download(t)) EXPECT_FLOAT_EQ(v, 1.0f);
    t.zero();
    for (float v : download(t)) EXPECT_FLOAT_EQ(v, 0.0f);
    tensor<bfloat16> b({3, 5});
    b.fill(__float2bfloat16(-2.5f));
    for (float v : download_f(b)) EXPECT_FLOAT_EQ(v, -2.5f);
    tensor<fp8_e4m3> q({7});
    q.fill(fp8_e4m3(0x3C));
    for (auto v : download(q)) EXPECT_EQ((int)v.bits, 0x3C);
}

// a failed runtime call the caller made earlier is not reported by the
// next C-ABI launch (the library resets the per-thread last error)
TEST_F(TensorTest, FillAfterFailedRuntimeCall) {
    int device_count = 0;
    (void)hipGetDeviceCount(&device_count);
    EXPECT_NE(hipSetDevice(device_count), hipSuccess);
    tensor<float> t({5});
    EXPECT_NO_THROW(t.fill(3.0f));
    for (float v : download(t)) EXPECT_FLOAT_EQ(v, 3.0f);
}

TEST_F(TensorTest, Reshape) {
    tensor<float> t({2, 2});
    std::vector<int> new_shape = {4, 1};
    t.reshape(new_shape);
    EXPECT_TRUE(t.shape() == new_shape);
    EXPECT_EQ(t.size(), 4);
    EXPECT_THROW(t.reshape({3, 2}), std::runtime_error);
}

TEST_F(TensorTest, MoveSemantics) {
    tensor<float> t1({2, 2});
    std::vector<float> host = {1.0f, 2.0f, 3.0f, 4.0f};
    t1.upload(host.data());
    tensor<float> t2(std::move(t1));
    EXPECT_EQ(t1.data(), nullptr);
    EXPECT_NE(t2.data(), nullptr);
    const auto back = download(t2);
    for (size_t i = 0; i < host.size(); ++i) EXPECT_FLOAT_EQ(host[i], back[i]);
    tensor<float> t3({2, 2});
    t3 = std::move(t2);
    EXPECT_EQ(t2.data(), nullptr);
    EXPECT_NE(t3.data(), nullptr);
}

TEST_F(TensorTest, Addition) {
    tensor<float> t1({2, 2}), t2({2, 2});
    std::vector<float> a = {1.0f, 2.0f, 3.0f, 4.0f}, b = {5.0f, 6.0f, 7.0f, 8.0f};
    t1.upload(a.data());
    t2.upload(b.data());
    tensor<float> t3 = t1 + t2;
    const auto r = download(t3);
    EXPECT_FLOAT_EQ(r[0], 6.0f);
    EXPECT_FLOAT_EQ(r[1], 8.0f);
    EXPECT_FLOAT_EQ(r[2], 10.0f);
    EXPECT_FLOAT_EQ(r[3], 12.0f);
}

TEST_F(TensorTest, InPlaceAddition) {
    tensor<float> t1({2, 2}), t2({2, 2});
    std::vector<float> a = {1.0f, 2.0f, 3.0f, 4.0f}, b = {5.0f, 6.0f, 7.0f, 8.0f};
    t1.upload(a.data());
    t2.upload(b.data());
    t1 += t2;
    const auto r = download(t1);
    EXPECT_FLOAT_EQ(r[0], 6.0f);
    EXPECT_FLOAT_EQ(r[1], 8.0f);
    EXPECT_FLOAT_EQ(r[2], 10.0f);
    EXPECT_FLOAT_EQ(r[3], 12.0f);
}

TEST_F(TensorTest, ShapeMismatchAddition) {
    tensor<float> t1({2, 2}), t2({2, 3});
    EXPECT_THROW(t1 + t2, std::runtime_error);
    EXPECT_THROW(t1 += t2, std::runtime_error);
}

TEST_F(TensorTest, Clone) {
    tensor<float> t1({2, 2});
    std::vector<float> host = {1.0f, 2.0f, 3.0f, 4.0f};
    t1.upload(host.data());
    tensor<float> t2 = t1.clone();
    EXPECT_TRUE(t2.shape() == t1.shape());
    EXPECT_NE(t2.data(), t1.data());
    const auto back = download(t2);
    for (size_t i = 0; i < host.size(); ++i) EXPECT_FLOAT_EQ(host[i], back[i]);
}

TEST_F(TensorTest, Equals) {
    tensor<float> t1({2, 2}), t2({2, 2}), t3({2, 2});
    std::vector<float> a = {1.0f, 2.0f, 3.0f, 4.0f}, b = {1.0f, 2.0f, 3.0f, 5.0f};
    t1.upload(a.data());
    t2.upload(a.data());
    t3.upload(b.data());
    EXPECT_TRUE(t1.equals(t2));
    EXPECT_FALSE(t1.equals(t3));
    const auto mask = download(t1 == t3);
    EXPECT_EQ((int)mask[0], 1);
    EXPECT_EQ((int)mask[3], 0);
}

TEST_F(TensorTest, ApproxEqual) {
    tensor<float> t1({2, 2}), t2({2, 2});
    std::vector<float> a = {1.0f, 2.0f, 3.0f, 4.0f}, b = {1.001f, 2.001f, 3.001f, 4.001f};
    t1.upload(a.data());
    t2.upload(b.data());
    EXPECT_TRUE(t1.approx_equal(t2, 0.01f));
    EXPECT_FALSE(t1.approx_equal(t2, 0.0001f));
}

TEST_F(TensorTest, SaveLoad) {
    tensor<float> t({3, 2});
    std::vector<float> host = {1, -2, 3.5f, 0, 7, -0.25f};
    t.upload(host.data());
    std::stringstream ss;
    t.save(ss);
    tensor<float> u({1});
    u.load(ss);
    EXPECT_TRUE(u.shape() == t.shape());
    EXPECT_TRUE(u.equals(t));
}

// ======================================================== Fp8TensorTest ==
// quantize / dequantize through the drop-in vs the oracle, bit for bit
TEST_F(Fp8TensorTest, QuantizeFloatMatchesOracle) {
    const int n = 4099;
    auto x = uniform(n, -3.0f, 3.0f, 11);
    x[0] = NAN;
    x[1] = INFINITY;
    x[2] = -INFINITY;
    x[3] = -0.0f;
    x[4] = 1e-30f;
    x[5] = 2.9999f * 1e6f;  // absmax well above the rest
    tensor<float> t({n});
    t.upload(x.data());
    for (int fmt : {DFO_E4M3, DFO_E5M2}) {
        const float s = dfo_scale(dfo_absmax_f32(x.data(), n), fmt);
        std::vector<uint8_t> expect(n);
        dfo_quantize_f32(x.data(), n, s, fmt, expect.data());
        std::vector<uint8_t> got(n);
        float got_s;
        if (fmt == DFO_E4M3) {
            auto q = quantize<fp8_e4m3>(t);
            q.download(reinterpret_cast<fp8_e4m3*>(got.data()));
            got_s = q.scale();
        } else {
            auto q = quantize<fp8_e5m2>(t);
            q.download(reinterpret_cast<fp8_e5m2*>(got.data()));
            got_s = q.scale();
        }
        EXPECT_EQ(got_s, s);
        int mismatches = 0;
        for (int i = 0; i < n; ++i) mismatches += got[i] != expect[i];
        EXPECT_EQ(mismatches, 0);
    }
}

TEST_F(Fp8TensorTest, QuantizeBFloat16MatchesOracle) {
    const int n = 1000;
    const auto xf = uniform(n, -50.0f, 50.0f, 12);
    const auto xh = float_to_bf16(xf);
    tensor<bfloat16> t({10, 100});
    t.upload(reinterpret_cast<const bfloat16*>(xh.data()));
    auto q = quantize<fp8_e5m2>(t);
    EXPECT_TRUE(q.shape() == t.shape());
    const float s = dfo_scale(dfo_absmax_bf16(xh.data(), n), DFO_E5M2);
    std::vector<uint8_t> expect(n), got(n);
    dfo_quantize_bf16(xh.data(), n, s, DFO_E5M2, expect.data());
    q.download(reinterpret_cast<fp8_e5m2*>(got.data()));
    EXPECT_EQ(q.scale(), s);
    EXPECT_TRUE(got == expect);
}

TEST_F(Fp8TensorTest, DequantizeMatchesOracle) {
    // every code, at a non-unit scale
    tensor<fp8_e4m3> q({256});
    std::vector<uint8_t> codes(256);
    for (int i = 0; i < 256; ++i) codes[i] = (uint8_t)i;
    q.upload(reinterpret_cast<const fp8_e4m3*>(codes.data()));
    q.set_scale(0.0371f);
    const auto f = download(dequantize<float>(q));
    const auto b = download_f(dequantize<bfloat16>(q));
    std::vector<float> ef(256);
    std::vector<uint16_t> eb(256);
    dfo_dequantize_f32(codes.data(), 256, 0.0371f, DFO_E4M3, ef.data());
    dfo_dequantize_bf16(codes.data(), 256, 0.0371f, DFO_E4M3, eb.data());
    int bad = 0;
    for (int i = 0; i < 256; ++i) {
        uint32_t a, e;
        std::memcpy(&a, &f[i], 4);
        std::memcpy(&e, &ef[i], 4);
        bad += a != e;
        const uint16_t bb = dfo_f32_to_bf16(b[i]);
        bad += bb != eb[i];
    }
    EXPECT_EQ(bad, 0);
}

TEST_F(Fp8TensorTest, RoundTripWithinHalfUlp) {
    const int n = 2048;
    const auto x = uniform(n, -1.0f, 1.0f, 13);
    tensor<float> t({n});
    t.upload(x.data());
    const auto back = download(dequantize<float>(quantize<fp8_e4m3>(t)));
    const float s = dfo_scale(dfo_absmax_f32(x.data(), n), DFO_E4M3);
    for (int i = 0; i < n; ++i) {
        // e4m3 has 3 fraction bits: |x - q| <= 2^-4 |x| in the normal
        // range, and <= 2^-10 * s (half the subnormal step) below it
        EXPECT_LE(std::fabs(back[i] - x[i]), std::max(std::fabs(x[i]) * 0.0625f, s * 0.0009766f) * 1.0001f);
    }
}

TEST_F(Fp8TensorTest, SaveLoadKeepsScale) {
    tensor<float> t({4, 4});
    const auto x = uniform(16, -9.0f, 9.0f, 14);
    t.upload(x.data());
    auto q = quantize<fp8_e4m3>(t);
    std::stringstream ss;
    q.save(ss);
    tensor<fp8_e4m3> r({1});
    r.load(ss);
    EXPECT_TRUE(r.equals(q));
    EXPECT_EQ(r.scale(), q.scale());
    EXPECT_THROW(q += r, std::runtime_error);
}

TEST_F(TensorTest, SaveKeepsTheReferenceLayout) {
    // int ndim, int dims[ndim], raw elements (dnn/core/tensor.cuh:104-125)
    tensor<float> t({2, 3});
    std::vector<float> host = {1, 2, 3, 4, 5, 6};
    t.upload(host.data());
    std::stringstream ss;
    t.save(ss);
    const std::string b = ss.str();
    ASSERT_EQ(b.size(), 4u + 8u + 24u);
    int hdr[3];
    std::memcpy(hdr, b.data(), sizeof(hdr));
    EXPECT_EQ(hdr[0], 2);
    EXPECT_EQ(hdr[1], 2);
    EXPECT_EQ(hdr[2], 3);
    EXPECT_EQ(std::memcmp(b.data() + 12, host.data(), 24), 0);
}

TEST_F(Fp8TensorTest, SaveWritesTaggedRecord) {
    tensor<float> t({5, 3});
    const auto x = uniform(15, -4.0f, 4.0f, 21);
    t.upload(x.data());
    auto q = quantize<fp8_e5m2>(t);
    std::stringstream ss;
    q.save(ss);
    const std::string b = ss.str();
    ASSERT_EQ(b.size(), 4u + 4u + 4u + 8u + 15u + 4u);
    int hdr[5];
    std::memcpy(hdr, b.data(), sizeof(hdr));
    EXPECT_LT(hdr[0], 0);                       // tag: never a valid ndim
    EXPECT_EQ(hdr[1], (int)DType::FP8E5M2);     // 6
    EXPECT_EQ(hdr[2], 2);
    EXPECT_EQ(hdr[3], 5);
    EXPECT_EQ(hdr[4], 3);
    float s;
    std::memcpy(&s, b.data() + b.size() - 4, 4);
    EXPECT_EQ(s, q.scale());
    // the other fp8 format refuses the record
    std::stringstream s2(b);
    tensor<fp8_e4m3> wrong({1});
    EXPECT_THROW(wrong.load(s2), std::runtime_error);
    // an integer tensor refuses it too
    std::stringstream s3(b);
    tensor<int> wrong_i({1});
    EXPECT_THROW(wrong_i.load(s3), std::runtime_error);
}

TEST_F(Fp8TensorTest, FloatTensorsLoadFp8RecordsDequantized) {
    tensor<float> t({7, 9});
    const auto x = uniform(63, -30.0f, 30.0f, 22);
    t.upload(x.data());
    auto q = quantize<fp8_e4m3>(t);
    std::stringstream ss;
    q.save(ss);
    const std::string b = ss.str();
    std::stringstream s1(b), s2(b);
    tensor<float> f({1});
    f.load(s1);
    EXPECT_TRUE(f.shape() == t.shape());
    EXPECT_TRUE(f.equals(dequantize<float>(q)));
    tensor<bfloat16> h({1});
    h.load(s2);
    EXPECT_TRUE(h.equals(dequantize<bfloat16>(q)));
}

TEST_F(Fp8TensorTest, LoadsUntaggedFp8Record) {
    // ndim, dims, codes, scale: the form written before the tag existed
    std::stringstream ss;
    const int ndim = 1, dim = 4;
    const uint8_t codes[4] = {0x38, 0xB8, 0x7E, 0x00};  // e4m3: 1, -1, 448, 0
    const float s = 0.5f;
    ss.write(reinterpret_cast<const char*>(&ndim), 4);
    ss.write(reinterpret_cast<const char*>(&dim), 4);
    ss.write(reinterpret_cast<const char*>(codes), 4);
    ss.write(reinterpret_cast<const char*>(&s), 4);
    tensor<fp8_e4m3> q({1});
    q.load(ss);
    EXPECT_EQ(q.scale(), 0.5f);
    const auto back = download(dequantize<float>(q));
    ASSERT_EQ(back.size(), 4u);
    EXPECT_EQ(back[0], 0.5f);
    EXPECT_EQ(back[1], -0.5f);
    EXPECT_EQ(back[2], 224.0f);
    EXPECT_EQ(back[3], 0.0f);
}

// ============================================== FullyConnectedLayerTest ==
TEST_F(FullyConnectedLayerTest, ConstructorAndInitialization) {
    const int in_features = 4, out_features = 3;
    FullyConnectedLayer<float> layer(in_features, out_features, true);
    auto params = layer.parameters();
    EXPECT_EQ(params.size(), 2u);
    EXPECT_EQ(params[0]->shape()[0], out_features);
    EXPECT_EQ(params[0]->shape()[1], in_features);
    EXPECT_EQ(params[1]->shape()[1], out_features);
    EXPECT_EQ(layer.name(), std::string("FullyConnected"));
    // Xavier uniform weights, zero bias
    const float limit = std::sqrt(6.0f / (in_features + out_features));
    for (float w : download(*params[0])) EXPECT_LE(std::fabs(w), limit);
    for (float b : download(*params[1])) EXPECT_EQ(b, 0.0f);
}

TEST_F(FullyConnectedLayerTest, ForwardPass) {
    const int in_features = 4, out_features = 3;
    FullyConnectedLayer<float> layer(in_features, out_features, true);
    tensor<float> input({1, in_features});
    std::vector<float> x(in_features);
    for (int i = 0; i < in_features; ++i) x[i] = static_cast<float>(i) / in_features;
    input.upload(x.data());
    auto params = layer.parameters();
    const auto w = download(*params[0]);
    const auto b = download(*params[1]);
    tensor<float> output = layer.forward(input);
    const auto y = download(output);

    std::vector<float> expect(out_features), exact(out_features);
    dfo_fc_forward(fp8_values(x, DFO_E4M3).data(), fp8_values(w, DFO_E4M3).data(), b.data(), expect.data(), 1,
                   in_features, out_features, 1);
    dfo_fc_forward(x.data(), w.data(), b.data(), exact.data(), 1, in_features, out_features, 1);
    for (int i = 0; i < out_features; ++i) {
        EXPECT_NEAR(y[i], expect[i], 1e-5);
        double bound = 0;  // two e4m3 roundings per product term
        for (int j = 0; j < in_features; ++j) bound += std::fabs(x[j] * w[i * in_features + j]);
        EXPECT_NEAR(y[i], exact[i], bound * (2 * 0.0625 + 0.0625 * 0.0625) + 1e-6);
    }
}

TEST_F(FullyConnectedLayerTest, BackwardPass) {
    const int in_features = 4, out_features = 3;
    FullyConnectedLayer<float> layer(in_features, out_features, true);
    tensor<float> input({1, in_features});
    std::vector<float> x(in_features);
    for (int i = 0; i < in_features; ++i) x[i] = static_cast<float>(i) / in_features;
    input.upload(x.data());
    tensor<float> output = layer.forward(input);
    tensor<float> grad_output(output.shape());
    std::vector<float> dy(out_features);
    for (int i = 0; i < out_features; ++i) dy[i] = static_cast<float>(i) / out_features;
    grad_output.upload(dy.data());
    auto params = layer.parameters();
    const auto w = download(*params[0]);
    tensor<float> grad_input = layer.backward(grad_output);
    const auto dx = download(grad_input);

    const auto dyd = fp8_values(dy, DFO_E5M2);
    std::vector<float> edx(in_features), edw(w.size()), edb(out_features);
    dfo_fc_backward_input(dyd.data(), fp8_values(w, DFO_E4M3).data(), edx.data(), 1, in_features, out_features, 1);
    dfo_fc_backward_weights(dyd.data(), fp8_values(x, DFO_E4M3).data(), edw.data(), 1, in_features, out_features, 1);
    dfo_fc_backward_bias(dy.data(), edb.data(), 1, out_features);
    for (int i = 0; i < in_features; ++i) EXPECT_NEAR(dx[i], edx[i], 1e-5);

    auto grads = layer.gradients();
    EXPECT_EQ(grads.size(), 2u);
    EXPECT_EQ(grads[0]->shape()[0], out_features);
    EXPECT_EQ(grads[0]->shape()[1], in_features);
    EXPECT_EQ(grads[1]->shape()[1], out_features);
    const auto dw = download(*grads[0]);
    const auto db = download(*grads[1]);
    for (size_t i = 0; i < dw.size(); ++i) EXPECT_NEAR(dw[i], edw[i], 1e-5);
    for (int i = 0; i < out_features; ++i) EXPECT_NEAR(db[i], edb[i], 1e-6);
}

TEST_F(FullyConnectedLayerTest, DifferentDimensions) {
    const int in_features = 5, out_features = 2;
    FullyConnectedLayer<float> layer(in_features, out_features, true);
    tensor<float> input({1, in_features});
    std::vector<float> x(in_features);
    for (int i = 0; i < in_features; ++i) x[i] = static_cast<float>(i) / in_features;
    input.upload(x.data());
    tensor<float> output = layer.forward(input);
    EXPECT_EQ(output.shape()[0], 1);
    EXPECT_EQ(output.shape()[1], out_features);
    tensor<float> grad_output(output.shape());
    std::vector<float> dy(out_features);
    for (int i = 0; i < out_features; ++i) dy[i] = static_cast<float>(i) / out_features;
    grad_output.upload(dy.data());
    tensor<float> grad_input = layer.backward(grad_output);
    EXPECT_EQ(grad_input.shape()[0], 1);
    EXPECT_EQ(grad_input.shape()[1], in_features);
}

TEST_F(FullyConnectedLayerTest, NonzeroInputGivesNonzeroOutput) {
    const int in_features = 2, out_features = 2;
    FullyConnectedLayer<float> layer(in_features, out_features, true);
    auto params = layer.parameters();
    std::vector<float> w = {1.0f, 2.0f, 3.0f, 4.0f};
    std::vector<float> b = {0.5f, -0.5f};
    params[0]->upload(w.data());
    params[1]->upload(b.data());
    tensor<float> input({1, in_features});
    std::vector<float> x = {1.0f, 2.0f};
    input.upload(x.data());
    const auto y = download(layer.forward(input));
    for (float v : y) EXPECT_NE(v, 0.0f);
    // fp8 values of W: 3 -> 336 * s ties to 320 * s (RNE), so y differs
    // from the fp32 {5.5, 10.5}; the oracle fixes what it must be
    std::vector<float> expect(2);
    dfo_fc_forward(fp8_values(x, DFO_E4M3).data(), fp8_values(w, DFO_E4M3).data(), b.data(), expect.data(), 1, 2, 2,
                   1);
    EXPECT_NEAR(y[0], expect[0], 1e-5);
    EXPECT_NEAR(y[1], expect[1], 1e-5);
}

TEST_F(FullyConnectedLayerTest, BackwardRequiresTrainingAndForward) {
    FullyConnectedLayer<float> inference(4, 3, false);
    tensor<float> g({1, 3});
    g.zero();
    EXPECT_THROW(inference.backward(g), std::runtime_error);
    FullyConnectedLayer<float> training(4, 3, true);
    EXPECT_THROW(training.backward(g), std::runtime_error);
    tensor<float> bad({1, 5});
    EXPECT_THROW(training.forward(bad), std::invalid_argument);
}

// ragged shapes (not multiples of 16) through forward and backward, fp32
TEST_F(FullyConnectedLayerTest, RaggedShapesMatchOracle) {
    const int N = 37, in_f = 100, out_f = 52;
    FullyConnectedLayer<float> layer(in_f, out_f, true);
    const auto w = uniform((size_t)out_f * in_f, -0.2f, 0.2f, 21);
    const auto b = uniform(out_f, -1.0f, 1.0f, 22);
    layer.parameters()[0]->upload(w.data());
    layer.parameters()[1]->upload(b.data());
    const auto x = uniform((size_t)N * in_f, -2.0f, 2.0f, 23);
    const auto dy = uniform((size_t)N * out_f, -0.01f, 0.01f, 24);
    tensor<float> input({N, in_f}), grad_out({N, out_f});
    input.upload(x.data());
    grad_out.upload(dy.data());
    const auto y = download(layer.forward(input));
    const auto dx = download(layer.backward(grad_out));
    const auto dw = download(*layer.grad_weights());
    const auto db = download(*layer.grad_bias());

    const auto xd = fp8_values(x, DFO_E4M3), wd = fp8_values(w, DFO_E4M3), dyd = fp8_values(dy, DFO_E5M2);
    std::vector<float> ey((size_t)N * out_f), edx((size_t)N * in_f), edw(w.size()), edb(out_f);
    dfo_fc_forward(xd.data(), wd.data(), b.data(), ey.data(), N, in_f, out_f, 4);
    dfo_fc_backward_input(dyd.data(), wd.data(), edx.data(), N, in_f, out_f, 4);
    dfo_fc_backward_weights(dyd.data(), xd.data(), edw.data(), N, in_f, out_f, 4);
    dfo_fc_backward_bias(dy.data(), edb.data(), N, out_f);
    EXPECT_LE(rel_err(y, ey), 1e-4);
    EXPECT_LE(rel_err(dx, edx), 1e-4);
    EXPECT_LE(rel_err(dw, edw), 1e-4);
    EXPECT_LE(rel_err(db, edb), 1e-5);
}

// Ten (tokens, in, out) triples drawn once from a fixed-seed mt19937: sizes
// below 1600 mixed with ones next to a 128- or 256-wide tile edge, through the
// layer's forward and backward (its caches, workspace and launch choices) and
// against the oracle on the fp8-dequantized operands.
TEST_F(FullyConnectedLayerTest, SeededShapeSweepMatchesOracle) {
    std::mt19937 gen(20261205u);
    auto draw = [&](int cap) {
        const uint32_t r = gen();
        if (r & 1u) return 1 + (int)((r >> 1) % (uint32_t)cap);
        const int edge = ((r >> 1) & 1u ? 128 : 256) * (1 + (int)((r >> 2) % 6u));
        return std::max(1, edge + (int)((r >> 5) % 3u) - 1);
    };
    for (int c = 0; c < 10; ++c) {
        const int N = draw(1024), in_f = draw(1600), out_f = draw(1024);
        SCOPED_TRACE("N=" + std::to_string(N) + " in=" + std::to_string(in_f) + " out=" + std::to_string(out_f));
        FullyConnectedLayer<float> layer(in_f, out_f, true);
        const auto w = uniform((size_t)out_f * in_f, -0.2f, 0.2f, 300 + c);
        const auto b = uniform(out_f, -1.0f, 1.0f, 400 + c);
        layer.parameters()[0]->upload(w.data());
        layer.parameters()[1]->upload(b.data());
        const auto x = uniform((size_t)N * in_f, -2.0f, 2.0f, 500 + c);
        const auto dy = uniform((size_t)N * out_f, -0.01f, 0.01f, 600 + c);
        tensor<float> input({N, in_f}), grad_out({N, out_f});
        input.upload(x.data());
        grad_out.upload(dy.data());
        const auto y = download(layer.forward(input));
        const auto dx = download(layer.backward(grad_out));
        const auto dw = download(*layer.grad_weights());
        const auto db = download(*layer.grad_bias());
        const auto xd = fp8_values(x, DFO_E4M3), wd = fp8_values(w, DFO_E4M3), dyd = fp8_values(dy, DFO_E5M2);
        std::vector<float> ey((size_t)N * out_f), edx((size_t)N * in_f), edw(w.size()), edb(out_f);
        dfo_fc_forward(xd.data(), wd.data(), b.data(), ey.data(), N, in_f, out_f, 8);
        dfo_fc_backward_input(dyd.data(), wd.data(), edx.data(), N, in_f, out_f, 8);
        dfo_fc_backward_weights(dyd.data(), xd.data(), edw.data(), N, in_f, out_f, 8);
        dfo_fc_backward_bias(dy.data(), edb.data(), N, out_f);
        EXPECT_LE(rel_err(y, ey), 1e-4);
        EXPECT_LE(rel_err(dx, edx), 1e-4);
        EXPECT_LE(rel_err(dw, edw), 1e-4);
        EXPECT_LE(rel_err(db, edb), 1e-5);
    }
}

// bfloat16 layer: operands quantized from bf16, outputs rounded to bf16
TEST_F(FullyConnectedLayerTest, BFloat16LayerMatchesOracle) {
    const int N = 64, in_f = 96, out_f = 80;
    FullyConnectedLayer<bfloat16> layer(in_f, out_f, true);
    const auto w = bf16_to_float(float_to_bf16(uniform((size_t)out_f * in_f, -0.3f, 0.3f, 31)));
    const auto b = bf16_to_float(float_to_bf16(uniform(out_f, -1.0f, 1.0f, 32)));
    const auto x = bf16_to_float(float_to_bf16(uniform((size_t)N * in_f, -3.0f, 3.0f, 33)));
    const auto dy = bf16_to_float(float_to_bf16(uniform((size_t)N * out_f, -0.5f, 0.5f, 34)));
    upload_bf16(*layer.weights(), w);
    upload_bf16(*layer.bias(), b);
    tensor<bfloat16> input({N, in_f}), grad_out({N, out_f});
    upload_bf16(input, x);
    upload_bf16(grad_out, dy);
    const auto y = download_f(layer.forward(input));
    const auto dx = download_f(layer.backward(grad_out));
    const auto dw = download_f(*layer.grad_weights());
    const auto db = download_f(*layer.grad_bias());

    const auto xd = fp8_values(x, DFO_E4M3), wd = fp8_values(w, DFO_E4M3), dyd = fp8_values(dy, DFO_E5M2);
    std::vector<float> ey((size_t)N * out_f), edx((size_t)N * in_f), edw(w.size()), edb(out_f);
    dfo_fc_forward(xd.data(), wd.data(), b.data(), ey.data(), N, in_f, out_f, 4);
    dfo_fc_backward_input(dyd.data(), wd.data(), edx.data(), N, in_f, out_f, 4);
    dfo_fc_backward_weights(dyd.data(), xd.data(), edw.data(), N, in_f, out_f, 4);
    dfo_fc_backward_bias(dy.data(), edb.data(), N, out_f);
    // bf16 outputs: unit roundoff 2^-8 (relative) on top of the fp32 bound
    const double tol = 1e-4 + 1.0 / 256;
    EXPECT_LE(rel_err(y, ey), tol);
    EXPECT_LE(rel_err(dx, edx), tol);
    EXPECT_LE(rel_err(dw, edw), tol);
    EXPECT_LE(rel_err(db, edb), tol);
}

// the FP16 layer (fully_connected_layer.cu:405): operands quantized from
// binary16, outputs the fp32 products rounded to nearest even binary16
TEST_F(FullyConnectedLayerTest, HalfLayerMatchesOracle) {
    const int N = 64, in_f = 96, out_f = 80;
    FullyConnectedLayer<__half> layer(in_f, out_f, true);
    const auto w = round_f16(uniform((size_t)out_f * in_f, -0.3f, 0.3f, 51));
    const auto b = round_f16(uniform(out_f, -1.0f, 1.0f, 52));
    const auto x = round_f16(uniform((size_t)N * in_f, -3.0f, 3.0f, 53));
    const auto dy = round_f16(uniform((size_t)N * out_f, -0.5f, 0.5f, 54));
    upload_f16(*layer.weights(), w);
    upload_f16(*layer.bias(), b);
    tensor<__half> input({N, in_f}), grad_out({N, out_f});
    upload_f16(input, x);
    upload_f16(grad_out, dy);
    const auto y = download_f(layer.forward(input));
    const auto dx = download_f(layer.backward(grad_out));
    const auto dw = download_f(*layer.grad_weights());
    const auto db = download_f(*layer.grad_bias());

    const auto xd = fp8_values(x, DFO_E4M3), wd = fp8_values(w, DFO_E4M3), dyd = fp8_values(dy, DFO_E5M2);
    std::vector<float> ey((size_t)N * out_f), edx((size_t)N * in_f), edw(w.size()), edb(out_f);
    dfo_fc_forward(xd.data(), wd.data(), b.data(), ey.data(), N, in_f, out_f, 4);
    dfo_fc_backward_input(dyd.data(), wd.data(), edx.data(), N, in_f, out_f, 4);
    dfo_fc_backward_weights(dyd.data(), xd.data(), edw.data(), N, in_f, out_f, 4);
    dfo_fc_backward_bias(dy.data(), edb.data(), N, out_f);
    // f16 outputs against the oracle's rounded to f16: the 1e-4 bar plus the
    // binary16 unit roundoff 2^-11 where the fp32 sums straddle a tie
    const double tol = 1e-4 + 1.0 / 2048;
    EXPECT_LE(rel_err(y, round_f16(ey)), tol);
    EXPECT_LE(rel_err(dx, round_f16(edx)), tol);
    EXPECT_LE(rel_err(dw, round_f16(edw)), tol);
    EXPECT_LE(rel_err(db, round_f16(edb)), tol);
}

// save_fp8 of an FP16 layer: e4m3 codes of the binary16 weights; load()
// gives the dequantized values rounded to binary16, the bias unchanged
TEST_F(FullyConnectedLayerTest, HalfSaveFp8RoundTrip) {
    const int in_f = 40, out_f = 24;
    FullyConnectedLayer<__half> a(in_f, out_f, false);
    const auto w = round_f16(uniform((size_t)out_f * in_f, -0.5f, 0.5f, 55));
    const auto b = round_f16(uniform(out_f, -1.0f, 1.0f, 56));
    upload_f16(*a.weights(), w);
    upload_f16(*a.bias(), b);
    std::stringstream ss;
    a.save_fp8(ss);
    FullyConnectedLayer<__half> c(in_f, out_f, false);
    c.load(ss);
    EXPECT_TRUE(download_f(*c.weights()) == round_f16(fp8_values(w, DFO_E4M3)));
    EXPECT_TRUE(download_f(*c.bias()) == b);
}

// all launches follow Hip::stream(): results on a created stream equal
// those on the legacy stream, bit for bit
TEST_F(FullyConnectedLayerTest, RunsOnTheCurrentStream) {
    const int N = 48, in_f = 64, out_f = 32;
    FullyConnectedLayer<float> layer(in_f, out_f, true);
    const auto x = uniform((size_t)N * in_f, -1.0f, 1.0f, 41);
    tensor<float> input({N, in_f});
    input.upload(x.data());
    const auto y0 = download(layer.forward(input));
    hipStream_t s;
    ASSERT_EQ(hipStreamCreate(&s), hipSuccess);
    std::vector<float> y1;
    {
        StreamGuard guard(s);
        EXPECT_EQ(Hip::stream(), s);
        y1 = download(layer.forward(input));
    }
    (void)hipStreamDestroy(s);
    EXPECT_TRUE(y0 == y1);
}

TEST_F(FullyConnectedLayerTest, SaveLoadRoundTrip) {
    FullyConnectedLayer<float> a(12, 7, false);
    std::stringstream ss;
    a.save(ss);
    FullyConnectedLayer<float> b(3, 3, false);
    b.load(ss);
    EXPECT_TRUE(b.weights()->equals(*a.weights()));
    EXPECT_TRUE(b.bias()->equals(*a.bias()));
    tensor<float> input({2, 12});
    input.fill(0.5f);
    EXPECT_TRUE(a.forward(input).equals(b.forward(input)));
}

TEST_F(FullyConnectedLayerTest, BackwardAfterLoadUsesLoadedWeights) {
    // The reference's backward reads weights_ at backward time and keeps its
    // input cache across load(): forward on layer a, load b's weights into a,
    // then backward equals a fresh layer with b's weights run forward +
    // backward on the same input (same X codes, same W codes, same dY).
    FullyConnectedLayer<float> a(48, 20, true), b(48, 20, true);
    tensor<float> input({8, 48}), grad({8, 20});
    const auto xi = uniform(8 * 48, -1.0f, 1.0f, 41), gi = uniform(8 * 20, -0.01f, 0.01f, 42);
    input.upload(xi.data());
    grad.upload(gi.data());
    a.forward(input);
    std::stringstream ss;
    b.save(ss);
    a.load(ss);
    const auto dxa = download(a.backward(grad));
    b.forward(input);
    const auto dxb = download(b.backward(grad));
    ASSERT_EQ(dxa.size(), dxb.size());
    for (size_t i = 0; i < dxa.size(); ++i) EXPECT_EQ(dxa[i], dxb[i]);
    EXPECT_TRUE(a.gradients()[0]->equals(*b.gradients()[0]));
    EXPECT_TRUE(a.gradients()[1]->equals(*b.gradients()[1]));
}

TEST_F(FullyConnectedLayerTest, SaveFp8LoadsDequantizedWeights) {
    FullyConnectedLayer<float> a(40, 24, false);
    std::stringstream full, small;
    a.save(full);
    a.save_fp8(small);
    // in, out, fp8 record of W (tag, dtype, ndim, dims, codes, scale), fp32 bias
    EXPECT_EQ(small.str().size(), 8u + (12u + 8u + 40u * 24u + 4u) + (4u + 16u + 24u * 4u));
    EXPECT_LT(small.str().size(), full.str().size() / 2);
    FullyConnectedLayer<float> b(3, 3, false);
    b.load(small);
    EXPECT_TRUE(b.weights()->shape() == a.weights()->shape());
    EXPECT_TRUE(b.weights()->equals(dequantize<float>(quantize<fp8_e4m3>(*a.weights()))));
    EXPECT_TRUE(b.bias()->equals(*a.bias()));
    // the reloaded layer quantizes its (dequantized) weights back to codes
    // within a step of the originals: the forward agrees to the fp8 bound
    tensor<float> input({4, 40});
    const auto xi = uniform(160, -1.0f, 1.0f, 31);
    input.upload(xi.data());
    const auto ya = download(a.forward(input)), yb = download(b.forward(input));
    float m = 0.0f, d = 0.0f;
    for (size_t i = 0; i < ya.size(); ++i) {
        m = std::max(m, std::fabs(ya[i]));
        d = std::max(d, std::fabs(ya[i] - yb[i]));
    }
    EXPECT_LE(d, 0.07f * m);
}

// ---- delayed scaling in the Linear layer ----
// values the GEMM sees when x is quantized at a given scale s (saturating)
std::vector<float> fp8_values_at(const std::vector<float>& x, float s, int fmt) {
    const int64_t n = (int64_t)x.size();
    std::vector<uint8_t> q(n);
    std::vector<float> d(n);
    dfo_quantize_f32(x.data(), n, s, fmt, q.data());
    dfo_dequantize_f32(q.data(), n, s, fmt, d.data());
    return d;
}

// The first step of a delayed-scaling layer seeds every history with the
// operand's own absmax: bit-identical to the just-in-time layer.
TEST_F(FullyConnectedLayerTest, DelayedScalingFirstStepEqualsJustInTime) {
    const int N = 70, in_f = 96, out_f = 40;
    FullyConnectedLayer<float> a(in_f, out_f, true), b(in_f, out_f, true);
    const auto w = uniform((size_t)out_f * in_f, -0.2f, 0.2f, 81);
    for (auto* l : {&a, &b}) l->parameters()[0]->upload(w.data());
    b.set_delayed_scaling(4);
    EXPECT_EQ(b.delayed_scaling(), 4);
    tensor<float> x({N, in_f}), gy({N, out_f});
    const auto xh = uniform((size_t)N * in_f, -1.0f, 1.0f, 82), gh = uniform((size_t)N * out_f, -0.1f, 0.1f, 83);
    x.upload(xh.data());
    gy.upload(gh.data());
    EXPECT_TRUE(download(a.forward(x)) == download(b.forward(x)));
    EXPECT_TRUE(download(a.backward(gy)) == download(b.backward(gy)));
    EXPECT_TRUE(download(*a.grad_weights()) == download(*b.grad_weights()));
    EXPECT_TRUE(download(*a.grad_bias()) == download(*b.grad_bias()));
}

// Later steps quantize at the scale of the history: an input that grew 4x
// saturates at 448 * (the earlier absmax / 448), and the history records
// both steps.
TEST_F(FullyConnectedLayerTest, DelayedScalingUsesHistoryScale) {
    const int N = 33, in_f = 64, out_f = 24;
    FullyConnectedLayer<float> layer(in_f, out_f, true);
    const auto w = uniform((size_t)out_f * in_f, -0.3f, 0.3f, 91);
    const auto bias = std::vector<float>(out_f, 0.0f);
    layer.parameters()[0]->upload(w.data());
    layer.set_delayed_scaling(2);
    const auto x1 = uniform((size_t)N * in_f, -1.0f, 1.0f, 92);
    auto x2 = uniform((size_t)N * in_f, -1.0f, 1.0f, 93);
    for (auto& v : x2) v *= 4.0f;
    tensor<float> t1({N, in_f}), t2({N, in_f});
    t1.upload(x1.data());
    t2.upload(x2.data());
    layer.forward(t1);
    const auto y2 = download(layer.forward(t2));
    // oracle: X at the scale of step 1's absmax, W at its own (unchanged) scale
    const float sx = dfo_scale(dfo_absmax_f32(x1.data(), (int64_t)x1.size()), DFO_E4M3);
    const auto xd = fp8_values_at(x2, sx, DFO_E4M3), wd = fp8_values(w, DFO_E4M3);
    std::vector<float> ey((size_t)N * out_f);
    dfo_fc_forward(xd.data(), wd.data(), bias.data(), ey.data(), N, in_f, out_f, 4);
    EXPECT_LE(rel_err(y2, ey), 1e-4);
    // the just-in-time result differs: the saturation is real
    const auto xj = fp8_values(x2, DFO_E4M3);
    std::vector<float> ej((size_t)N * out_f);
    dfo_fc_forward(xj.data(), wd.data(), bias.data(), ej.data(), N, in_f, out_f, 4);
    EXPECT_GT(rel_err(y2, ej), 1e-2);
    std::vector<float> h(2);
    CHECK_HIP_EX(hipMemcpy(h.data(), layer.amax_history(0), 2 * sizeof(float), hipMemcpyDeviceToHost));
    EXPECT_EQ(h[0], dfo_absmax_f32(x2.data(), (int64_t)x2.size()));
    EXPECT_EQ(h[1], dfo_absmax_f32(x1.data(), (int64_t)x1.size()));
}

// load() between two training forwards of a delayed-scaling layer: the
// second forward writes the W^T codes of the loaded weights at the delayed
// W scale (the history still holds the old weights' absmax), and the
// backward's dX must use those codes with that same scale.
TEST_F(FullyConnectedLayerTest, DelayedScalingForwardAfterLoadKeepsWtScale) {
    const int N = 16, in_f = 64, out_f = 24;
    FullyConnectedLayer<float> layer(in_f, out_f, true), other(in_f, out_f, true);
    const auto w_old = uniform((size_t)out_f * in_f, -0.3f, 0.3f, 111);
    const auto w_new = uniform((size_t)out_f * in_f, -0.1f, 0.1f, 112);
    layer.parameters()[0]->upload(w_old.data());
    other.parameters()[0]->upload(w_new.data());
    layer.set_delayed_scaling(16);
    tensor<float> x({N, in_f}), gy({N, out_f});
    const auto xh = uniform((size_t)N * in_f, -1.0f, 1.0f, 113), gh = uniform((size_t)N * out_f, -0.01f, 0.01f, 114);
    x.upload(xh.data());
    gy.upload(gh.data());
    layer.forward(x);
    std::stringstream ss;
    other.save(ss);
    layer.load(ss);
    layer.forward(x);
    const auto dx = download(layer.backward(gy));
    // oracle: W (loaded) at the delayed scale of the old weights' absmax; dY
    // at its own scale (the first backward seeds its history)
    const float sw = dfo_scale(dfo_absmax_f32(w_old.data(), (int64_t)w_old.size()), DFO_E4M3);
    const auto wd = fp8_values_at(w_new, sw, DFO_E4M3), gd = fp8_values(gh, DFO_E5M2);
    std::vector<float> e((size_t)N * in_f);
    dfo_fc_backward_input(gd.data(), wd.data(), e.data(), N, in_f, out_f, 4);
    EXPECT_LE(rel_err(dx, e), 1e-4);
}

// ---- LayerNormLayer (dnn/layers/layer_norm_layer.cu) and the fused producer ----
TEST_F(LayerNormLayerTest, ForwardMatchesOracle) {
    const int rows = 37, C = 100;
    LayerNormLayer<float> ln(C, 1e-5f, true, false);
    EXPECT_EQ(ln.parameters().size(), 2u);
    const auto g = uniform(C, 0.5f, 1.5f, 101), b = uniform(C, -1.0f, 1.0f, 102);
    ln.parameters()[0]->upload(g.data());
    ln.parameters()[1]->upload(b.data());
    const auto x = uniform((size_t)rows * C, -3.0f, 3.0f, 103);
    tensor<float> t({rows, C});
    t.upload(x.data());
    const auto y = download(ln.forward(t));
    std::vector<float> e(x.size());
    dfo_layernorm(x.data(), rows, C, g.data(), b.data(), 1e-5f, 0, e.data());
    EXPECT_LE(rel_err(y, e), 1e-5);
}

TEST_F(LayerNormLayerTest, DefaultParametersAreIdentityAffine) {
    const int rows = 8, C = 1600;  // GPT-2 XL width: beyond a 1024-thread block per row
    LayerNormLayer<float> a(C), b(C, 1e-5f, false);
    EXPECT_TRUE(b.parameters().empty());
    const auto x = uniform((size_t)rows * C, -2.0f, 2.0f, 104);
    tensor<float> t({rows, C});
    t.upload(x.data());
    EXPECT_TRUE(download(a.forward(t)) == download(b.forward(t)));
    std::vector<float> e(x.size());
    dfo_layernorm(x.data(), rows, C, nullptr, nullptr, 1e-5f, 0, e.data());
    EXPECT_LE(rel_err(download(b.forward(t)), e), 1e-5);
}

TEST_F(LayerNormLayerTest, BackwardPassesTheGradientThrough) {
    LayerNormLayer<float> ln(16, 1e-5f, true, true);
    tensor<float> g({4, 16});
    const auto gh = uniform(64, -1.0f, 1.0f, 105);
    g.upload(gh.data());
    bool threw = false;
    try {
        ln.backward(g);
    } catch (const std::runtime_error&) {
        threw = true;
    }
    EXPECT_TRUE(threw);  // training mode, no forward yet
    ln.forward(g);
    EXPECT_TRUE(download(ln.backward(g)) == gh);
}

TEST_F(LayerNormLayerTest, SaveLoadRoundTrip) {
    LayerNormLayer<float> a(24), b(24);
    const auto g = uniform(24, 0.5f, 1.5f, 106);
    a.parameters()[0]->upload(g.data());
    std::stringstream ss;
    a.save(ss);
    b.load(ss);
    EXPECT_TRUE(download(*b.parameters()[0]) == g);
}

TEST_F(LayerNormLayerTest, BFloat16MatchesOracle) {
    const int rows = 20, C = 96;
    LayerNormLayer<bfloat16> ln(C);
    const auto x = bf16_to_float(float_to_bf16(uniform((size_t)rows * C, -2.0f, 2.0f, 107)));
    tensor<bfloat16> t({rows, C});
    upload_bf16(t, x);
    const auto y = download_f(ln.forward(t));
    std::vector<float> e(x.size());
    dfo_layernorm(x.data(), rows, C, nullptr, nullptr, 1e-5f, 1, e.data());
    EXPECT_LE(rel_err(y, e), 1e-2);  // one bf16 step where the binary32 sums differ in order
}

TEST_F(LayerNormLayerTest, HalfMatchesOracle) {
    const int rows = 20, C = 96;
    LayerNormLayer<__half> ln(C);
    const auto x = round_f16(uniform((size_t)rows * C, -2.0f, 2.0f, 108));
    tensor<__half> t({rows, C});
    upload_f16(t, x);
    const auto y = download_f(ln.forward(t));
    std::vector<float> e(x.size());
    dfo_layernorm(x.data(), rows, C, nullptr, nullptr, 1e-5f, 0, e.data());
    EXPECT_LE(rel_err(y, round_f16(e)), 2e-3);  // one binary16 step where the sums differ in order
}

// fc.forward(x, ln) == fc.forward(ln.forward(x)), forward and backward, just
// in time and with delayed scaling
TEST_F(FullyConnectedLayerTest, LayerNormFusedEqualsUnfused) {
    const int N = 48, in_f = 160, out_f = 72;
    for (int hist : {0, 4}) {
        FullyConnectedLayer<float> a(in_f, out_f, true), b(in_f, out_f, true);
        const auto w = uniform((size_t)out_f * in_f, -0.2f, 0.2f, 111);
        for (auto* l : {&a, &b}) {
            l->parameters()[0]->upload(w.data());
            l->set_delayed_scaling(hist);
        }
        LayerNormLayer<float> ln(in_f, 1e-5f, true, true);
        const auto g = uniform(in_f, 0.5f, 1.5f, 112), bb = uniform(in_f, -0.5f, 0.5f, 113);
        ln.parameters()[0]->upload(g.data());
        ln.parameters()[1]->upload(bb.data());
        for (int step = 0; step < 2; ++step) {
            auto xh = uniform((size_t)N * in_f, -2.0f, 2.0f, 114 + step);
            tensor<float> x({N, in_f}), gy({N, out_f});
            x.upload(xh.data());
            const auto gh = uniform((size_t)N * out_f, -0.1f, 0.1f, 120 + step);
            gy.upload(gh.data());
            const auto ya = download(a.forward(ln.forward(x)));
            const auto yb = download(b.forward(x, ln));
            EXPECT_TRUE(ya == yb);
            EXPECT_TRUE(download(a.backward(gy)) == download(b.backward(gy)));
            EXPECT_TRUE(download(*a.grad_weights()) == download(*b.grad_weights()));
        }
    }
}

// fc1 -> fc2 chained as the reference block's MLP runs them
// (transformer_block.cu:79-81, :127-134): fc2.forward(fc1, x) and
// fc1.backward(fc2, gy) equal the unfused pairs bit for bit -- output, input
// gradient, both layers' weight and bias gradients -- over two training
// steps, for float, bf16 and binary16 layers, on a small shape (the fused
// GEMMs' two-pass form) and on one whose fc1 output takes the persistent
// kernel that folds the absmax; with delayed scaling on the layers they are
// the unfused pairs.
template <typename TT>
std::vector<float> chain_dl(const tensor<TT>& t) {
    if constexpr (std::is_same_v<TT, float>) return download(t);
    else return download_f(t);
}

template <typename TT>
void chain_up(tensor<TT>& t, const std::vector<float>& v) {
    if constexpr (std::is_same_v<TT, float>) t.upload(v.data());
    else if constexpr (std::is_same_v<TT, __half>) upload_f16(t, v);
    else upload_bf16(t, v);
}

template <typename TT>
void chain_case(int N, int in_f, int hid, int out_f, int hist, uint64_t seed) {
    SCOPED_TRACE("N=" + std::to_string(N) + " " + std::to_string(in_f) + "->" + std::to_string(hid) + "->" +
                 std::to_string(out_f) + " hist=" + std::to_string(hist));
    FullyConnectedLayer<TT> a1(in_f, hid, true), a2(hid, out_f, true), b1(in_f, hid, true), b2(hid, out_f, true);
    const auto w1 = uniform((size_t)hid * in_f, -0.1f, 0.1f, seed), w2 = uniform((size_t)out_f * hid, -0.05f, 0.05f,
                                                                                  seed + 1);
    const auto c1 = uniform(hid, -0.5f, 0.5f, seed + 2), c2 = uniform(out_f, -0.5f, 0.5f, seed + 3);
    for (auto* l : {&a1, &b1}) {
        chain_up(*l->weights(), w1);
        chain_up(*l->bias(), c1);
        l->set_delayed_scaling(hist);
    }
    for (auto* l : {&a2, &b2}) {
        chain_up(*l->weights(), w2);
        chain_up(*l->bias(), c2);
        l->set_delayed_scaling(hist);
    }
    for (int step = 0; step < 2; ++step) {
        tensor<TT> x({N, in_f}), gy({N, out_f});
        chain_up(x, uniform((size_t)N * in_f, -2.0f, 2.0f, seed + 10 + step));
        chain_up(gy, uniform((size_t)N * out_f, -0.1f, 0.1f, seed + 20 + step));
        EXPECT_TRUE(chain_dl(a2.forward(a1.forward(x))) == chain_dl(b2.forward(b1, x)));
        EXPECT_TRUE(chain_dl(a1.backward(a2.backward(gy))) == chain_dl(b1.backward(b2, gy)));
        EXPECT_TRUE(chain_dl(*a1.grad_weights()) == chain_dl(*b1.grad_weights()));
        EXPECT_TRUE(chain_dl(*a2.grad_weights()) == chain_dl(*b2.grad_weights()));
        EXPECT_TRUE(chain_dl(*a1.grad_bias()) == chain_dl(*b1.grad_bias()));
        EXPECT_TRUE(chain_dl(*a2.grad_bias()) == chain_dl(*b2.grad_bias()));
    }
}

TEST_F(FullyConnectedLayerTest, ChainedPairEqualsUnfused) {
    chain_case<float>(48, 160, 96, 72, 0, 300);
    chain_case<bfloat16>(48, 160, 96, 72, 0, 310);
    chain_case<float>(48, 160, 96, 72, 4, 320);
    chain_case<float>(4096, 512, 4096, 512, 0, 330);
    chain_case<bfloat16>(4096, 512, 4096, 512, 0, 340);
    chain_case<__half>(48, 160, 96, 72, 0, 350);
    chain_case<__half>(4096, 512, 4096, 512, 0, 360);
}

TEST_F(FullyConnectedLayerTest, ChainedPairChecksSizes) {
    FullyConnectedLayer<float> a(16, 32, true), b(48, 8, true);
    tensor<float> x({4, 16});
    EXPECT_THROW(b.forward(a, x), std::invalid_argument);
    tensor<float> g({4, 8});
    EXPECT_THROW(a.backward(b, g), std::invalid_argument);
}

// A chained forward refused for its input's shape leaves the layer as it
// was: the backward that follows uses the last completed forward (its cached
// X^T codes were neither replaced nor resized).
TEST_F(FullyConnectedLayerTest, RefusedChainedForwardKeepsTheLayer) {
    FullyConnectedLayer<float> a(16, 32, true), b(32, 8, true);
    tensor<float> x({4, 16}), g({4, 8});
    x.upload(uniform(64, -1.0f, 1.0f, 950).data());
    g.upload(uniform(32, -1.0f, 1.0f, 951).data());
    (void)b.forward(a, x);
    const auto dx = download(b.backward(g));
    const auto dw = download(*b.grad_weights());
    tensor<float> x3({4, 4, 16}), wide({4, 17});
    EXPECT_THROW(b.forward(a, x3), std::invalid_argument);
    EXPECT_THROW(b.forward(a, wide), std::invalid_argument);
    EXPECT_TRUE(download(b.backward(g)) == dx);
    EXPECT_TRUE(download(*b.grad_weights()) == dw);
}

// An empty batch: forward gives [0, out], backward gives [0, in] and zero
// weight and bias gradients (sums over no rows), alone and chained.
TEST_F(FullyConnectedLayerTest, EmptyBatchForwardBackward) {
    FullyConnectedLayer<float> a(16, 32, true), b(32, 8, true);
    tensor<float> x({4, 16}), g({4, 8});
    x.upload(uniform(64, -1.0f, 1.0f, 960).data());
    g.upload(uniform(32, -1.0f, 1.0f, 961).data());
    (void)b.forward(a, x);  // non-zero gradients first
    (void)a.backward(b, g);
    tensor<float> x0({0, 16}), g0({0, 8});
    EXPECT_TRUE(b.forward(a, x0).shape() == std::vector<int>({0, 8}));
    EXPECT_TRUE(a.backward(b, g0).shape() == std::vector<int>({0, 16}));
    for (auto* l : {&a, &b}) {
        for (float v : download(*l->grad_weights())) EXPECT_EQ(v, 0.0f);
        for (float v : download(*l->grad_bias())) EXPECT_EQ(v, 0.0f);
    }
    EXPECT_TRUE(a.forward(x0).shape() == std::vector<int>({0, 32}));
    tensor<float> gh0({0, 32});
    EXPECT_TRUE(a.backward(gh0).shape() == std::vector<int>({0, 16}));
    tensor<float> gbad({1, 32});
    EXPECT_THROW(a.backward(gbad), std::invalid_argument);
}

// ---- AdamOptimizer: the reference's cases (adam_optimizer_test.cu:21-214),
// plus exact agreement with the oracle's step ----
TEST_F(AdamOptimizerTest, BasicUpdate) {
    tensor<float> param1({2, 2}), param2({2, 2}), grad1({2, 2}), grad2({2, 2});
    param1.fill(1.0f);
    param2.fill(2.0f);
    grad1.fill(0.1f);
    grad2.fill(0.2f);
    AdamOptimizer<float> optimizer(0.001f);
    optimizer.update_parameters({&param1, &param2}, {&grad1, &grad2});
    optimizer.step();
    EXPECT_LT(download(param1)[0], 1.0f);
    EXPECT_LT(download(param2)[0], 2.0f);
}

TEST_F(AdamOptimizerTest, MomentumAndRMS) {
    tensor<float> param({2, 2}), grad({2, 2});
    param.fill(1.0f);
    grad.fill(0.1f);
    AdamOptimizer<float> optimizer(0.001f, 0.9f, 0.999f);
    optimizer.update_parameters({&param}, {&grad});
    optimizer.step();
    const float first = download(param)[0];
    optimizer.step();
    EXPECT_NE(first, download(param)[0]);
}

TEST_F(AdamOptimizerTest, WeightDecay) {
    tensor<float> param({2, 2}), grad({2, 2});
    param.fill(1.0f);
    grad.fill(0.1f);
    AdamOptimizer<float> optimizer(0.001f, 0.9f, 0.999f, 1e-8f, 0.1f);
    optimizer.update_parameters({&param}, {&grad});
    optimizer.step();
    EXPECT_GT(1.0f - download(param)[0], 0.0f);
}

TEST_F(AdamOptimizerTest, ZeroGrad) {
    tensor<float> param({2, 2}), grad({2, 2});
    param.fill(1.0f);
    grad.fill(0.1f);
    AdamOptimizer<float> optimizer(0.001f);
    optimizer.update_parameters({&param}, {&grad});
    optimizer.zero_grad();
    for (float g : download(grad)) EXPECT_EQ(g, 0.0f);
}

TEST_F(AdamOptimizerTest, LearningRateChange) {
    tensor<float> param({2, 2}), grad({2, 2});
    param.fill(1.0f);
    grad.fill(0.1f);
    AdamOptimizer<float> optimizer(0.001f);
    optimizer.update_parameters({&param}, {&grad});
    optimizer.step();
    const float first = download(param)[0];
    optimizer.set_learning_rate(0.002f);
    optimizer.step();
    const float second = download(param)[0];
    EXPECT_GT(std::abs(second - first), std::abs(first - 1.0f));
}

TEST_F(AdamOptimizerTest, ParameterUpdate) {
    tensor<float> param1({2, 2}), grad1({2, 2});
    param1.fill(1.0f);
    grad1.fill(0.1f);
    AdamOptimizer<float> optimizer(0.001f);
    optimizer.update_parameters({&param1}, {&grad1});
    optimizer.step();
    const float first = download(param1)[0];
    tensor<float> new_param({2, 2}), new_grad({2, 2});
    new_param.fill(3.0f);
    new_grad.fill(0.3f);
    optimizer.update_parameters({&new_param}, {&new_grad});
    optimizer.step();
    EXPECT_EQ(download(param1)[0], first);
    EXPECT_NE(download(new_param)[0], 3.0f);
}

// A Linear layer's parameters through three steps, against the oracle's
// element-by-element restatement, bit for bit.
TEST_F(AdamOptimizerTest, LinearLayerStepsMatchOracle) {
    FullyConnectedLayer<float> fc(96, 40, true);
    tensor<float> x({33, 96});
    const auto xh = uniform(33 * 96, -1.0f, 1.0f, 41);
    x.upload(xh.data());
    tensor<float> gy({33, 40});
    const auto gyh = uniform(33 * 40, -1.0f, 1.0f, 42);
    gy.upload(gyh.data());
    AdamOptimizer<float> opt(0.01f, 0.9f, 0.999f, 1e-8f, 0.01f);
    opt.update_parameters(fc.parameters(), fc.gradients());
    std::vector<std::vector<float>> p, m, v;
    for (auto* t : fc.parameters()) {
        p.push_back(download(*t));
        m.emplace_back(t->size(), 0.0f);
        v.emplace_back(t->size(), 0.0f);
    }
    for (int step = 1; step <= 3; ++step) {
        fc.forward(x);
        fc.backward(gy);
        const auto grads = fc.gradients();
        std::vector<std::vector<float>> g;
        for (auto* t : grads) g.push_back(download(*t));
        opt.step();
        for (size_t i = 0; i < p.size(); ++i)
            dfo_adam_step(p[i].data(), g[i].data(), m[i].data(), v[i].data(), (int64_t)p[i].size(), 0.01f, 0.9f,
                          0.999f, 1e-8f, 0.01f, step, 1.0f);
    }
    const auto params = fc.parameters();
    for (size_t i = 0; i < p.size(); ++i) {
        EXPECT_TRUE(download(*params[i]) == p[i]);
        EXPECT_TRUE(download(opt.first_moment(params[i])) == m[i]);
        EXPECT_TRUE(download(opt.second_moment(params[i])) == v[i]);
    }
    EXPECT_EQ(opt.timestep(), 3);
}

// step_clipped(max_norm) == clip_grad_norm(grads, max_norm) + step(), except
// that the gradients keep their values.
TEST_F(AdamOptimizerTest, StepClippedEqualsClipThenStep) {
    std::vector<std::unique_ptr<tensor<float>>> pa, pb, ga, gb;
    const int sizes[3] = {5000, 8192 * 3 + 7, 12};
    for (int i = 0; i < 3; ++i) {
        const auto ph = uniform(sizes[i], -1.0f, 1.0f, 50 + i);
        const auto gh = uniform(sizes[i], -2.0f, 2.0f, 60 + i);
        for (auto* vec : {&pa, &pb}) {
            vec->push_back(std::make_unique<tensor<float>>(std::vector<int>{sizes[i]}));
            vec->back()->upload(ph.data());
        }
        for (auto* vec : {&ga, &gb}) {
            vec->push_back(std::make_unique<tensor<float>>(std::vector<int>{sizes[i]}));
            vec->back()->upload(gh.data());
        }
    }
    auto raw = [](std::vector<std::unique_ptr<tensor<float>>>& v) {
        std::vector<tensor<float>*> r;
        for (auto& t : v) r.push_back(t.get());
        return r;
    };
    auto pra = raw(pa), prb = raw(pb), gra = raw(ga), grb = raw(gb);
    AdamOptimizer<float> a(0.001f), b(0.001f);
    a.update_parameters(pra, gra);
    b.update_parameters(prb, grb);
    const auto g0 = download(*ga[1]);
    utils::clip_grad_norm(gra, 1.0f);
    a.step();
    b.step_clipped(1.0f);
    for (int i = 0; i < 3; ++i) EXPECT_TRUE(download(*pa[i]) == download(*pb[i]));
    EXPECT_TRUE(download(*gb[1]) == g0);   // fused: gradients unchanged
    EXPECT_FALSE(download(*ga[1]) == g0);  // reference order: clipped in place
}

// ---- clip_grad_norm (clip_grad_norm.cu:31-62) ----
TEST_F(ClipGradNormTest, ScalesWhenAboveMaxNorm) {
    tensor<float> a({1}), b({1});
    const float three = 3.0f, four = 4.0f;
    a.upload(&three);
    b.upload(&four);
    std::vector<tensor<float>*> grads{&a, &b};
    utils::clip_grad_norm(grads, 1.0f);
    const float f = 1.0f / 5.0f;
    EXPECT_EQ(download(a)[0], 3.0f * f);
    EXPECT_EQ(download(b)[0], 4.0f * f);
}

TEST_F(ClipGradNormTest, LeavesGradientsAtOrBelowMaxNorm) {
    tensor<float> a({1}), b({1});
    const float three = 3.0f, four = 4.0f;
    a.upload(&three);
    b.upload(&four);
    std::vector<tensor<float>*> grads{&a, &b};
    utils::clip_grad_norm(grads, 5.0f);
    EXPECT_EQ(download(a)[0], 3.0f);
    utils::clip_grad_norm(grads, 6.0f);
    EXPECT_EQ(download(b)[0], 4.0f);
}

TEST_F(ClipGradNormTest, MatchesOracleOnLayerGradients) {
    FullyConnectedLayer<float> fc(300, 200, true);
    tensor<float> x({64, 300}), gy({64, 200});
    const auto xh = uniform(64 * 300, -1.0f, 1.0f, 71), gh = uniform(64 * 200, -1.0f, 1.0f, 72);
    x.upload(xh.data());
    gy.upload(gh.data());
    fc.forward(x);
    fc.backward(gy);
    auto grads = fc.gradients();
    std::vector<std::vector<float>> host;
    for (auto* t : grads) host.push_back(download(*t));
    const float* ptrs[2] = {host[0].data(), host[1].data()};
    const int64_t n[2] = {(int64_t)host[0].size(), (int64_t)host[1].size()};
    const float norm = dfo_grad_norm(ptrs, n, 2);
    EXPECT_GT(norm, 1.0f);
    utils::clip_grad_norm(grads, 1.0f);
    for (int i = 0; i < 2; ++i) {
        dfo_clip_scale(host[i].data(), n[i], norm, 1.0f);
        EXPECT_TRUE(download(*grads[i]) == host[i]);
    }
}

int main(int argc, char** argv) {
    const int rc = mini_test::run_all(argc, argv);
#ifdef DNN_TESTS_SKIP_TEARDOWN
    // The sanitized build (make asan) ends here, once every result is
    // printed: at static teardown the ROCm runtime's own finalizers free
    // memory after the runtime has unloaded, which the sanitizer's device
    // allocator aborts on.
    std::cout.flush();
    std::_Exit(rc);
#endif
    return rc;
}
