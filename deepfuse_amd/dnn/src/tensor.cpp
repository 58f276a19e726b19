// dnn::tensor<TT> (dnn/core/tensor.cu:76-498 in the reference) and the fp8
// quantize / dequantize conversions, with all device work through the C ABI.
#include "dnn/core/tensor.hpp"

#include <cstring>
#include <sstream>
#include <stdexcept>
#include <type_traits>

#include "dnn/core/hip.hpp"
#include "dnn/utils/common.hpp"

namespace dnn {

namespace {

void* stream_arg() { return reinterpret_cast<void*>(Hip::stream()); }

template <typename TT>
constexpr bool is_fp8() {
    return dtype_traits<TT>::is_fp8;
}

// host value of an element as float (for equals on 16-bit float types)
template <typename TT>
float host_float(const TT& v) {
    if constexpr (std::is_same_v<TT, __half>) return __half2float(v);
    else if constexpr (std::is_same_v<TT, bfloat16>) return __bfloat162float(v);
    else return static_cast<float>(v);
}

}  // namespace

template <typename TT>
tensor<TT>::tensor(const std::vector<int>& shape) : shape_(shape) {
    int64_t total = 1;
    for (int d : shape) {
        if (d < 0) throw std::invalid_argument("tensor: negative dimension");
        total *= d;
    }
    if (total > INT32_MAX) throw std::invalid_argument("tensor: more than 2^31-1 elements");
    total_size_ = static_cast<int>(total);
    if (total_size_ > 0) CHECK_HIP_EX(hipMalloc(&data_, (size_t)total_size_ * sizeof(TT)));
    if constexpr (is_fp8<TT>()) {
        CHECK_HIP_EX(hipMalloc(&scale_, 256));
        const float one = 1.0f;
        CHECK_HIP_EX(hipMemcpy(scale_, &one, sizeof(float), hipMemcpyHostToDevice));
    }
}

template <typename TT>
tensor<TT>::~tensor() {
    if (data_) (void)hipFree(data_);
    if (scale_) (void)hipFree(scale_);
}

template <typename TT>
void tensor<TT>::upload(const TT* host_data) {
    if (total_size_ == 0) return;
    CHECK_HIP_EX(hipStreamSynchronize(Hip::stream()));
    CHECK_HIP_EX(hipMemcpy(data_, host_data, (size_t)total_size_ * sizeof(TT), hipMemcpyHostToDevice));
}

template <typename TT>
void tensor<TT>::download(TT* host_data) const {
    if (total_size_ == 0) return;
    CHECK_HIP_EX(hipStreamSynchronize(Hip::stream()));
    CHECK_HIP_EX(hipMemcpy(host_data, data_, (size_t)total_size_ * sizeof(TT), hipMemcpyDeviceToHost));
}

template <typename TT>
int tensor<TT>::size(int dim) const {
    if (dim < 0 || dim >= static_cast<int>(shape_.size())) throw std::out_of_range("Dimension out of range");
    return shape_[dim];
}

template <typename TT>
tensor<TT>& tensor<TT>::reshape(const std::vector<int>& new_shape) {
    int64_t total = 1;
    for (int d : new_shape) total *= d;
    if (total != total_size_) {
        std::ostringstream oss;
        oss << "reshape: size mismatch, current=" << to_string() << " new=[";
        for (size_t i = 0; i < new_shape.size(); ++i) oss << new_shape[i] << (i + 1 < new_shape.size() ? "," : "");
        oss << "]";
        throw std::runtime_error(oss.str());
    }
    shape_ = new_shape;
    return *this;
}

template <typename TT>
tensor<TT>& tensor<TT>::fill(TT value) {
    CHECK_DF_EX(df_fill(data_, total_size_, (int)sizeof(TT), &value, stream_arg()));
    return *this;
}

template <typename TT>
tensor<TT>& tensor<TT>::zero() {
    TT z;
    std::memset(static_cast<void*>(&z), 0, sizeof(TT));
    return fill(z);
}

template <typename TT>
tensor<TT>::tensor(tensor&& other) noexcept
    : shape_(std::move(other.shape_)), data_(other.data_), total_size_(other.total_size_), scale_(other.scale_) {
    other.data_ = nullptr;
    other.scale_ = nullptr;
    other.total_size_ = 0;
    other.shape_.clear();
}

template <typename TT>
tensor<TT>& tensor<TT>::operator=(tensor&& other) noexcept {
    if (this != &other) {
        if (data_) (void)hipFree(data_);
        if (scale_) (void)hipFree(scale_);
        shape_ = std::move(other.shape_);
        data_ = other.data_;
        scale_ = other.scale_;
        total_size_ = other.total_size_;
        other.data_ = nullptr;
        other.scale_ = nullptr;
        other.total_size_ = 0;
        other.shape_.clear();
    }
    return *this;
}

template <typename TT>
tensor<TT> tensor<TT>::clone() const {
    tensor<TT> out(shape_);
    if (total_size_ > 0)
        CHECK_HIP_EX(hipMemcpyAsync(out.data_, data_, (size_t)total_size_ * sizeof(TT), hipMemcpyDeviceToDevice,
                                    Hip::stream()));
    if (scale_)
        CHECK_HIP_EX(hipMemcpyAsync(out.scale_, scale_, sizeof(float), hipMemcpyDeviceToDevice, Hip::stream()));
    return out;
}

template <typename TT>
tensor<TT>& tensor<TT>::operator+=(const tensor<TT>& other) {
    if (shape_ != other.shape()) throw std::runtime_error("Shape mismatch in operator+=");
    if constexpr (is_fp8<TT>()) throw std::runtime_error("operator+= is not defined for fp8 tensors");
    CHECK_DF_EX(df_add(dtype_traits<TT>::value, data_, other.data_, data_, total_size_, stream_arg()));
    return *this;
}

template <typename TT>
tensor<TT> operator+(const tensor<TT>& a, const tensor<TT>& b) {
    if (a.shape() != b.shape()) throw std::runtime_error("Shape mismatch in operator+");
    if constexpr (dtype_traits<TT>::is_fp8) throw std::runtime_error("operator+ is not defined for fp8 tensors");
    tensor<TT> out(a.shape());
    CHECK_DF_EX(df_add(dtype_traits<TT>::value, a.data(), b.data(), out.data(), a.size(), stream_arg()));
    return out;
}

template <typename TT>
tensor<uint8_t> tensor<TT>::operator==(const tensor<TT>& other) const {
    if (shape_ != other.shape_) throw std::invalid_argument("Shape mismatch in operator==");
    tensor<uint8_t> out(shape_);
    CHECK_DF_EX(df_equal_mask(dtype_traits<TT>::value, data_, other.data_, out.data(), total_size_, stream_arg()));
    return out;
}

template <typename TT>
bool tensor<TT>::equals(const tensor<TT>& other) const {
    if (shape_ != other.shape_ || total_size_ != other.total_size_) return false;
    std::vector<TT> a(total_size_), b(total_size_);
    download(a.data());
    other.download(b.data());
    for (int i = 0; i < total_size_; ++i) {
        if constexpr (is_fp8<TT>()) {
            if (a[i] != b[i]) return false;
        } else if (host_float(a[i]) != host_float(b[i])) {
            return false;
        }
    }
    if constexpr (is_fp8<TT>()) return scale() == other.scale();
    return true;
}

template <typename TT>
bool tensor<TT>::approx_equal(const tensor<TT>& other, float atol) const {
    if (shape_ != other.shape_ || total_size_ != other.total_size_) return false;
    if constexpr (is_fp8<TT>()) throw std::runtime_error("approx_equal is not defined for fp8 tensors");
    tensor<uint8_t> mask(shape_);
    CHECK_DF_EX(df_approx_equal_mask(dtype_traits<TT>::value, data_, other.data_, mask.data(), total_size_, atol,
                                     stream_arg()));
    std::vector<uint8_t> host(total_size_);
    mask.download(host.data());
    for (uint8_t v : host)
        if (v == 0) return false;
    return true;
}

template <typename TT>
std::string tensor<TT>::to_string() const {
    std::ostringstream oss;
    oss << "tensor: [";
    for (size_t i = 0; i < shape_.size(); ++i) oss << shape_[i] << (i + 1 < shape_.size() ? ", " : "");
    oss << "]";
    return oss.str();
}

template <typename TT>
float tensor<TT>::scale() const {
    if (!scale_) throw std::runtime_error("scale() is defined for fp8 tensors only");
    float s = 0.0f;
    CHECK_HIP_EX(hipStreamSynchronize(Hip::stream()));
    CHECK_HIP_EX(hipMemcpy(&s, scale_, sizeof(float), hipMemcpyDeviceToHost));
    return s;
}

template <typename TT>
void tensor<TT>::set_scale(float s) {
    if (!scale_) throw std::runtime_error("set_scale() is defined for fp8 tensors only");
    CHECK_HIP_EX(hipStreamSynchronize(Hip::stream()));
    CHECK_HIP_EX(hipMemcpy(scale_, &s, sizeof(float), hipMemcpyHostToDevice));
}

// On-disk layout.  Element types the reference has keep its layout
// unchanged -- int ndim, int dims[ndim], raw elements (tensor.cuh:104-125) --
// so files move both ways.  fp8 tensors, which have no counterpart there,
// write a tagged record: int kFp8Tag (negative, so never a valid ndim), int
// dtype (DType::FP8E4M3 = 5 / FP8E5M2 = 6), int ndim, int dims[ndim], one code
// per element, float scale.  An fp8 tensor also loads the untagged form (ndim,
// dims, codes, scale) that earlier builds wrote; a float or bfloat16 tensor
// loads a tagged fp8 record as its dequantized values (decode(code) * scale).
namespace {
constexpr int32_t kFp8Tag = -0x38465044;

template <typename Q>
tensor<Q> read_fp8_body(std::istream& in, const std::vector<int>& shape) {
    tensor<Q> q(shape);
    std::vector<Q> host(q.size());
    in.read(reinterpret_cast<char*>(host.data()), (std::streamsize)host.size());
    float s = 1.0f;
    in.read(reinterpret_cast<char*>(&s), sizeof(s));
    if (!in) throw std::runtime_error("tensor::load: truncated fp8 record");
    q.upload(host.data());
    q.set_scale(s);
    return q;
}
}  // namespace

template <typename TT>
void tensor<TT>::save(std::ostream& out) const {
    if constexpr (is_fp8<TT>()) {
        const int32_t tag = kFp8Tag, dt = dtype_traits<TT>::value;
        out.write(reinterpret_cast<const char*>(&tag), sizeof(tag));
        out.write(reinterpret_cast<const char*>(&dt), sizeof(dt));
    }
    const int ndim = static_cast<int>(shape_.size());
    out.write(reinterpret_cast<const char*>(&ndim), sizeof(ndim));
    out.write(reinterpret_cast<const char*>(shape_.data()), ndim * sizeof(int));
    std::vector<TT> host(total_size_);
    download(host.data());
    out.write(reinterpret_cast<const char*>(host.data()), (std::streamsize)total_size_ * sizeof(TT));
    if constexpr (is_fp8<TT>()) {
        const float s = scale();
        out.write(reinterpret_cast<const char*>(&s), sizeof(s));
    }
}

template <typename TT>
void tensor<TT>::load(std::istream& in) {
    int first = 0;
    in.read(reinterpret_cast<char*>(&first), sizeof(first));
    if (!in) throw std::runtime_error("tensor::load: bad header");
    int fp8_dtype = -1;
    if (first == kFp8Tag) {
        in.read(reinterpret_cast<char*>(&fp8_dtype), sizeof(fp8_dtype));
        in.read(reinterpret_cast<char*>(&first), sizeof(first));
        if (!in || (fp8_dtype != DF_DTYPE_FP8E4M3 && fp8_dtype != DF_DTYPE_FP8E5M2))
            throw std::runtime_error("tensor::load: bad fp8 record header");
    }
    const int ndim = first;
    if (ndim < 0 || ndim > 16) throw std::runtime_error("tensor::load: bad header");
    std::vector<int> shape(ndim);
    in.read(reinterpret_cast<char*>(shape.data()), ndim * sizeof(int));
    if (!in) throw std::runtime_error("tensor::load: truncated header");
    if (fp8_dtype >= 0) {
        if constexpr (is_fp8<TT>()) {
            if (fp8_dtype != dtype_traits<TT>::value)
                throw std::runtime_error("tensor::load: the file holds the other fp8 format");
            *this = read_fp8_body<TT>(in, shape);
        } else if constexpr (std::is_same_v<TT, float> || std::is_same_v<TT, bfloat16> ||
                             std::is_same_v<TT, __half>) {
            if (fp8_dtype == DF_DTYPE_FP8E4M3)
                *this = dequantize<TT>(read_fp8_body<fp8_e4m3>(in, shape));
            else
                *this = dequantize<TT>(read_fp8_body<fp8_e5m2>(in, shape));
        } else {
            throw std::runtime_error(
                "tensor::load: an fp8 record loads into fp8, float, __half or bfloat16 tensors only");
        }
        return;
    }
    *this = tensor<TT>(shape);
    std::vector<TT> host(total_size_);
    in.read(reinterpret_cast<char*>(host.data()), (std::streamsize)total_size_ * sizeof(TT));
    if (!in) throw std::runtime_error("tensor::load: truncated data");
    upload(host.data());
    if constexpr (is_fp8<TT>()) {
        float s = 1.0f;
        in.read(reinterpret_cast<char*>(&s), sizeof(s));
        if (!in) throw std::runtime_error("tensor::load: missing fp8 scale");
        set_scale(s);
    }
}

// ------------------------------------------------------------ conversions --
template <typename Q, typename T>
tensor<Q> quantize(const tensor<T>& x) {
    static_assert(dtype_traits<Q>::is_fp8, "quantize<Q>: Q must be fp8_e4m3 or fp8_e5m2");
    static_assert(std::is_same_v<T, float> || std::is_same_v<T, bfloat16> || std::is_same_v<T, __half>,
                  "quantize: float, __half or bfloat16 input");
    constexpr int fmt = dtype_traits<Q>::fmt;
    if constexpr (std::is_same_v<T, __half>) {
        // binary16 widens to binary32 exactly: the codes and scale of the
        // widened copy are those of the binary16 values
        tensor<float> wide(x.shape());
        CHECK_DF_EX(df_convert(DF_DTYPE_HALF, x.data(), DF_DTYPE_FLOAT32, wide.data(), x.size(), stream_arg()));
        return quantize<Q>(wide);
    }
    tensor<Q> q(x.shape());
    const int64_t n = x.size();
    const size_t ws_bytes = df_absmax_workspace_bytes();
    tensor<uint8_t> ws({(int)ws_bytes});
    void* st = stream_arg();
    uint8_t* codes = reinterpret_cast<uint8_t*>(q.data());
    if constexpr (std::is_same_v<T, __half>) {
        // handled above
    } else if constexpr (std::is_same_v<T, float>) {
        CHECK_DF_EX(df_absmax_scale_f32(x.data(), n, fmt, nullptr, q.scale_data(), ws.data(), ws_bytes, st));
        if (fmt == DF_FMT_E4M3) CHECK_DF_EX(df_quantize_f32_e4m3(x.data(), n, q.scale_data(), codes, st));
        else CHECK_DF_EX(df_quantize_f32_e5m2(x.data(), n, q.scale_data(), codes, st));
    } else {
        const uint16_t* xb = reinterpret_cast<const uint16_t*>(x.data());
        CHECK_DF_EX(df_absmax_scale_bf16(xb, n, fmt, nullptr, q.scale_data(), ws.data(), ws_bytes, st));
        if (fmt == DF_FMT_E4M3) CHECK_DF_EX(df_quantize_bf16_e4m3(xb, n, q.scale_data(), codes, st));
        else CHECK_DF_EX(df_quantize_bf16_e5m2(xb, n, q.scale_data(), codes, st));
    }
    CHECK_HIP_EX(hipStreamSynchronize(Hip::stream()));  // ws is released on return
    return q;
}

template <typename T, typename Q>
tensor<T> dequantize(const tensor<Q>& q) {
    static_assert(dtype_traits<Q>::is_fp8, "dequantize<T, Q>: Q must be fp8_e4m3 or fp8_e5m2");
    constexpr int fmt = dtype_traits<Q>::fmt;
    if constexpr (std::is_same_v<T, __half>) {
        // code * scale in binary32, then rounded to nearest even binary16
        const tensor<float> wide = dequantize<float>(q);
        tensor<__half> out(q.shape());
        CHECK_DF_EX(df_convert(DF_DTYPE_FLOAT32, wide.data(), DF_DTYPE_HALF, out.data(), q.size(), stream_arg()));
        CHECK_HIP_EX(hipStreamSynchronize(Hip::stream()));  // wide is released on return
        return out;
    }
    tensor<T> out(q.shape());
    const int64_t n = q.size();
    const uint8_t* codes = reinterpret_cast<const uint8_t*>(q.data());
    void* st = stream_arg();
    if constexpr (std::is_same_v<T, float>) {
        if (fmt == DF_FMT_E4M3) CHECK_DF_EX(df_dequantize_e4m3_f32(codes, n, q.scale_data(), out.data(), st));
        else CHECK_DF_EX(df_dequantize_e5m2_f32(codes, n, q.scale_data(), out.data(), st));
    } else if constexpr (!std::is_same_v<T, __half>) {
        static_assert(std::is_same_v<T, bfloat16>, "dequantize: float, __half or bfloat16 output");
        uint16_t* ob = reinterpret_cast<uint16_t*>(out.data());
        if (fmt == DF_FMT_E4M3) CHECK_DF_EX(df_dequantize_e4m3_bf16(codes, n, q.scale_data(), ob, st));
        else CHECK_DF_EX(df_dequantize_e5m2_bf16(codes, n, q.scale_data(), ob, st));
    }
    return out;
}

#define DF_INSTANTIATE(T)   \
    template struct tensor<T>; \
    template tensor<T> operator+(const tensor<T>&, const tensor<T>&);
DF_INSTANTIATE(float)
DF_INSTANTIATE(__half)
DF_INSTANTIATE(bfloat16)
DF_INSTANTIATE(int8_t)
DF_INSTANTIATE(uint8_t)
DF_INSTANTIATE(int)
DF_INSTANTIATE(fp8_e4m3)
DF_INSTANTIATE(fp8_e5m2)
#undef DF_INSTANTIATE

template tensor<fp8_e4m3> quantize<fp8_e4m3, float>(const tensor<float>&);
template tensor<fp8_e5m2> quantize<fp8_e5m2, float>(const tensor<float>&);
template tensor<fp8_e4m3> quantize<fp8_e4m3, bfloat16>(const tensor<bfloat16>&);
template tensor<fp8_e5m2> quantize<fp8_e5m2, bfloat16>(const tensor<bfloat16>&);
template tensor<float> dequantize<float, fp8_e4m3>(const tensor<fp8_e4m3>&);
template tensor<float> dequantize<float, fp8_e5m2>(const tensor<fp8_e5m2>&);
template tensor<bfloat16> dequantize<bfloat16, fp8_e4m3>(const tensor<fp8_e4m3>&);
template tensor<bfloat16> dequantize<bfloat16, fp8_e5m2>(const tensor<fp8_e5m2>&);
template tensor<fp8_e4m3> quantize<fp8_e4m3, __half>(const tensor<__half>&);
template tensor<fp8_e5m2> quantize<fp8_e5m2, __half>(const tensor<__half>&);
template tensor<__half> dequantize<__half, fp8_e4m3>(const tensor<fp8_e4m3>&);
template tensor<__half> dequantize<__half, fp8_e5m2>(const tensor<fp8_e5m2>&);

}  // namespace dnn
