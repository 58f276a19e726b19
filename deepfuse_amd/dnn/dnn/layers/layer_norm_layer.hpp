// dnn/layers/layer_norm_layer.hpp -- LayerNorm of the drop-in, the producer
// of the qkv and fc1 Linears' input.
//
// Same interface and forward math as the reference's LayerNormLayer<T>
// (dnn/layers/layer_norm_layer.cuh, .cu:8-131): per row of norm_size values,
// y = (x - mean) / sqrt(var + eps) [* gamma + beta], gamma = 1 and beta = 0
// at construction; backward returns a copy of the incoming gradient (the
// reference's backward, .cu:82-90), after checking the training-mode cache;
// save/load write norm_size, gamma, beta, grad_gamma, grad_beta.
// Provided for float and bfloat16 (the Linear path's element types).
//
// One deliberate difference: the input is normalised in runs of norm_size
// values (rows = size / norm_size), whatever its rank.  The reference takes
// shape[0] rows of shape[1] values (.cu:70-71), which for the [B, T, E]
// tensors of its TransformerBlock normalises over T instead of E, and it
// launches norm_size threads per block, which fails beyond 1024 (GPT-2 XL's
// 1600).
//
// The fused producer: FullyConnectedLayer::forward(input, norm) quantizes
// LayerNorm(input) straight into the Linear's fp8 operands without
// materialising the normalised tensor.
#pragma once

#include <iostream>
#include <optional>
#include <string>
#include <vector>

#include "dnn/core/layer.hpp"
#include "dnn/core/tensor.hpp"

namespace dnn {

template <typename T>
class LayerNormLayer : public Layer<T> {
public:
    LayerNormLayer(int norm_size, float epsilon = 1e-5f, bool affine = true, bool training_enabled = false);
    ~LayerNormLayer() override;

    tensor<T> forward(const tensor<T>& input) override;
    tensor<T> backward(const tensor<T>& grad_output) override;

    std::vector<tensor<T>*> parameters() override;
    std::vector<tensor<T>*> gradients() override;

    std::string name() const override { return "LayerNorm"; }

    void save(std::ostream& out) const override;
    void load(std::istream& in) override;

    int norm_size() const { return norm_size_; }
    float epsilon() const { return epsilon_; }
    bool affine() const { return affine_; }
    const tensor<T>& gamma() const { return gamma_; }
    const tensor<T>& beta() const { return beta_; }
    // rows of `input` (size / norm_size); throws when it does not divide
    int rows_of(const tensor<T>& input) const;
    // what forward() records for backward in training mode (a copy of the
    // input), for callers that consume the normalised values fused
    void note_input(const tensor<T>& input);

private:
    int norm_size_;
    float epsilon_;
    bool affine_;
    tensor<T> gamma_;
    tensor<T> beta_;
    tensor<T> grad_gamma_;
    tensor<T> grad_beta_;
    std::optional<tensor<T>> input_cache_;
    void* ws_ = nullptr;  // row statistics (device), grown on demand
    size_t ws_bytes_ = 0;
};

}  // namespace dnn
