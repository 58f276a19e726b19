// dnn/core/layer.hpp -- layer interfaces of the drop-in.
//
// Same virtual interface as the reference (dnn/core/layer.cuh:17-94), so
// that layers and models written against it compile unchanged: BaseLayer
// (name, save, load), LayerAsymmetric<TTO, TTI> (forward, backward with the
// layer's own cached input, parameters, gradients, training flag) and
// LayerWeightBiasAsymmetric (owned weights, bias and their gradients).
#pragma once

#include <iostream>
#include <string>
#include <utility>
#include <vector>

#include "dnn/core/tensor.hpp"

namespace dnn {

class BaseLayer {
public:
    virtual ~BaseLayer() = default;
    virtual std::string name() const = 0;
    virtual void save(std::ostream& out) const = 0;
    virtual void load(std::istream& in) = 0;
};

template <typename TTO, typename TTI>
class LayerAsymmetric : public BaseLayer {
public:
    explicit LayerAsymmetric(bool training_enabled = false) : training_enabled_(training_enabled) {}
    ~LayerAsymmetric() override = default;

    virtual tensor<TTO> forward(const tensor<TTI>& input) = 0;
    virtual tensor<TTO> backward(const tensor<TTO>& grad_output) = 0;
    virtual std::vector<tensor<TTO>*> parameters() { return {}; }
    virtual std::vector<tensor<TTO>*> gradients() { return {}; }
    bool training_enabled() const { return training_enabled_; }

protected:
    bool training_enabled_;
};

template <typename TTO, typename TTI>
class LayerWeightBiasAsymmetric : public LayerAsymmetric<TTO, TTI> {
public:
    LayerWeightBiasAsymmetric(tensor<TTO>&& weights, tensor<TTO>&& bias, tensor<TTO>&& grad_weights,
                              tensor<TTO>&& grad_bias, bool training_enabled = false)
        : LayerAsymmetric<TTO, TTI>(training_enabled),
          weights_(std::move(weights)),
          bias_(std::move(bias)),
          grad_weights_(std::move(grad_weights)),
          grad_bias_(std::move(grad_bias)) {}
    ~LayerWeightBiasAsymmetric() override = default;

    tensor<TTO>* weights() { return &weights_; }
    tensor<TTO>* bias() { return &bias_; }
    tensor<TTO>* grad_weights() { return &grad_weights_; }
    tensor<TTO>* grad_bias() { return &grad_bias_; }

    virtual void initialize_weights() = 0;

    std::vector<tensor<TTO>*> parameters() override { return {&weights_, &bias_}; }
    std::vector<tensor<TTO>*> gradients() override { return {&grad_weights_, &grad_bias_}; }
    tensor<TTO> backward(const tensor<TTO>& grad_output) override = 0;

protected:
    tensor<TTO> weights_;
    tensor<TTO> bias_;
    tensor<TTO> grad_weights_;
    tensor<TTO> grad_bias_;
};

template <typename TT>
using Layer = LayerAsymmetric<TT, TT>;

template <typename TT>
using LayerWeightBias = LayerWeightBiasAsymmetric<TT, TT>;

}  // namespace dnn
