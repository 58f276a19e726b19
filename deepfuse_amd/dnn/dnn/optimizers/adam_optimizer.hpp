// dnn/optimizers/adam_optimizer.hpp -- Adam for the C++ drop-in.
//
// The reference's AdamOptimizer<T> (dnn/optimizers/adam_optimizer.cuh,
// adam_optimizer.cu:83-130): per-parameter first and second moments created
// zero-filled by update_parameters, step() increments the step count and
// updates every listed parameter (coupled L2 weight decay, bias-corrected
// moments).  Provided for T = float, the element type of the Linear layer's
// weight and bias gradients; one df_adam_update_f32 call updates the whole
// list (the reference launches one kernel per tensor).
//
// Addition: step_clipped(max_norm) is utils::clip_grad_norm(gradients(),
// max_norm) followed by step(), with the clip factor applied inside the
// update instead of rewriting the gradients (they keep their unclipped
// values); the decision to clip is taken on the device, so neither call
// synchronises the host.
#pragma once

#include <memory>
#include <unordered_map>

#include "dnn/optimizers/optimizer.hpp"

namespace dnn {

template <typename T>
class AdamOptimizer : public Optimizer<T> {
public:
    AdamOptimizer(T learning_rate = 0.001, T beta1 = 0.9, T beta2 = 0.999, T epsilon = 1e-8,
                  T weight_decay = 0.0)
        : learning_rate_(learning_rate), beta1_(beta1), beta2_(beta2), epsilon_(epsilon),
          weight_decay_(weight_decay), timestep_(0) {}

    void step() override;
    void zero_grad() override;
    void update_parameters(const std::vector<tensor<T>*>& parameters,
                           const std::vector<tensor<T>*>& gradients) override;

    T learning_rate() const override { return learning_rate_; }
    void set_learning_rate(T new_lr) override { learning_rate_ = new_lr; }

    // clip_grad_norm(gradients(), max_norm) + step() in one pass over the
    // gradients; returns the device pointer of the norm it computed.
    const float* step_clipped(float max_norm);
    int timestep() const { return timestep_; }
    tensor<T>& first_moment(tensor<T>* param) { return *m_.at(param); }
    tensor<T>& second_moment(tensor<T>* param) { return *v_.at(param); }

private:
    void launch(const float* clip_norm, float max_norm);

    T learning_rate_, beta1_, beta2_, epsilon_, weight_decay_;
    int timestep_;
    std::unordered_map<tensor<T>*, std::unique_ptr<tensor<T>>> m_;
    std::unordered_map<tensor<T>*, std::unique_ptr<tensor<T>>> v_;
    std::unique_ptr<tensor<float>> norm_;
    std::unique_ptr<tensor<uint8_t>> ws_;
};

}  // namespace dnn
