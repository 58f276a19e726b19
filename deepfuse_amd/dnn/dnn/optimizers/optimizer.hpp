// dnn/optimizers/optimizer.hpp -- optimizer interface of the C++ drop-in.
//
// Same interface as the reference's Optimizer<T> (dnn/optimizers/optimizer.cuh:
// step, zero_grad, the parameter and gradient lists, update_parameters, the
// learning rate).
#pragma once

#include <vector>

#include "dnn/core/tensor.hpp"

namespace dnn {

template <typename T>
class Optimizer {
public:
    virtual ~Optimizer() = default;

    virtual void step() = 0;
    virtual void zero_grad() = 0;

    virtual std::vector<tensor<T>*>& parameters() { return parameters_; }
    virtual const std::vector<tensor<T>*>& parameters() const { return parameters_; }
    virtual std::vector<tensor<T>*>& gradients() { return gradients_; }
    virtual const std::vector<tensor<T>*>& gradients() const { return gradients_; }

    virtual void update_parameters(const std::vector<tensor<T>*>& parameters,
                                   const std::vector<tensor<T>*>& gradients) {
        parameters_ = parameters;
        gradients_ = gradients;
    }

    virtual T learning_rate() const = 0;
    virtual void set_learning_rate(T new_lr) = 0;

protected:
    std::vector<tensor<T>*> parameters_;
    std::vector<tensor<T>*> gradients_;
};

}  // namespace dnn
