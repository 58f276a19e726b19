// LayerNormLayer<T> of the drop-in (the reference's
// dnn/layers/layer_norm_layer.cu:8-131), device work through df_layernorm on
// Hip::stream().
#include "dnn/layers/layer_norm_layer.hpp"

#include <stdexcept>

#include "dnn/core/hip.hpp"
#include "dnn/utils/common.hpp"

namespace dnn {

namespace {
inline void* st() { return reinterpret_cast<void*>(Hip::stream()); }
}  // namespace

template <typename T>
LayerNormLayer<T>::LayerNormLayer(int norm_size, float epsilon, bool affine, bool training_enabled)
    : Layer<T>(training_enabled),
      norm_size_(norm_size),
      epsilon_(epsilon),
      affine_(affine),
      gamma_({norm_size}),
      beta_({norm_size}),
      grad_gamma_({norm_size}),
      grad_beta_({norm_size}) {
    if (norm_size <= 0) throw std::invalid_argument("LayerNormLayer: norm_size must be positive");
    if (affine_) {
        gamma_.fill(static_cast<T>(1.0f));
        beta_.fill(static_cast<T>(0.0f));
    }
}

template <typename T>
LayerNormLayer<T>::~LayerNormLayer() {
    if (ws_) (void)hipFree(ws_);
}

template <typename T>
int LayerNormLayer<T>::rows_of(const tensor<T>& input) const {
    if (input.size() % norm_size_ != 0)
        throw std::invalid_argument("LayerNormLayer: input of " + std::to_string(input.size()) +
                                    " values is not a whole number of rows of " + std::to_string(norm_size_));
    return input.size() / norm_size_;
}

template <typename T>
void LayerNormLayer<T>::note_input(const tensor<T>& input) {
    if (this->training_enabled_) input_cache_ = input.clone();
}

template <typename T>
tensor<T> LayerNormLayer<T>::forward(const tensor<T>& input) {
    const int rows = rows_of(input);
    note_input(input);
    tensor<T> output(input.shape());
    if (rows == 0) return output;
    const size_t need = df_layernorm_workspace_bytes(rows, norm_size_, 0, 0);
    if (need > ws_bytes_) {
        if (ws_) {
            CHECK_HIP_EX(hipStreamSynchronize(Hip::stream()));
            CHECK_HIP_EX(hipFree(ws_));
            ws_ = nullptr;
        }
        CHECK_HIP_EX(hipMalloc(&ws_, need));
        ws_bytes_ = need;
    }
    CHECK_DF_EX(df_layernorm(dtype_traits<T>::value, input.data(), rows, norm_size_, norm_size_,
                             affine_ ? gamma_.data() : nullptr, affine_ ? beta_.data() : nullptr, epsilon_,
                             output.data(), norm_size_, ws_, ws_bytes_, st()));
    return output;
}

// the reference's backward (.cu:82-90): the incoming gradient, copied
template <typename T>
tensor<T> LayerNormLayer<T>::backward(const tensor<T>& grad_output) {
    if (this->training_enabled_ && !input_cache_.has_value())
        throw std::runtime_error("LayerNormLayer: input_cache_ is empty in backward().");
    return grad_output.clone();
}

template <typename T>
std::vector<tensor<T>*> LayerNormLayer<T>::parameters() {
    return affine_ ? std::vector<tensor<T>*>{&gamma_, &beta_} : std::vector<tensor<T>*>{};
}

template <typename T>
std::vector<tensor<T>*> LayerNormLayer<T>::gradients() {
    return affine_ ? std::vector<tensor<T>*>{&grad_gamma_, &grad_beta_} : std::vector<tensor<T>*>{};
}

template <typename T>
void LayerNormLayer<T>::save(std::ostream& out) const {
    out.write(reinterpret_cast<const char*>(&norm_size_), sizeof(norm_size_));
    gamma_.save(out);
    beta_.save(out);
    grad_gamma_.save(out);
    grad_beta_.save(out);
}

template <typename T>
void LayerNormLayer<T>::load(std::istream& in) {
    in.read(reinterpret_cast<char*>(&norm_size_), sizeof(norm_size_));
    gamma_.load(in);
    beta_.load(in);
    grad_gamma_.load(in);
    grad_beta_.load(in);
}

template class LayerNormLayer<float>;
template class LayerNormLayer<__half>;
template class LayerNormLayer<bfloat16>;

}  // namespace dnn
