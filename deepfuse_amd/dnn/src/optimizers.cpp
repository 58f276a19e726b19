// optimizers.cpp -- AdamOptimizer<float> and utils::clip_grad_norm<float> of
// the C++ drop-in, on df_adam_update_f32 / df_clip_grad_norm_f32.
//
// Reference: dnn/optimizers/adam_optimizer.cu:83-130 and
// dnn/utils/clip_grad_norm.cu:31-62.
#include <stdexcept>
#include <vector>

#include "dnn/core/hip.hpp"
#include "dnn/core/tensor.hpp"
#include "dnn/optimizers/adam_optimizer.hpp"
#include "dnn/utils/common.hpp"

namespace dnn {
namespace {

void* stream_arg() { return reinterpret_cast<void*>(Hip::stream()); }

// Per-thread device scratch for the norm: the block partials (grown on
// demand) and the norm itself.  Work on one thread's stream is ordered, so
// reusing them call after call is safe.
struct NormScratch {
    void* ws = nullptr;
    size_t bytes = 0;
    float* norm = nullptr;
    int device = -1;
    ~NormScratch() {
        if (ws) (void)hipFree(ws);
        if (norm) (void)hipFree(norm);
    }
    void reserve(size_t need) {
        int dev = 0;
        CHECK_HIP_EX(hipGetDevice(&dev));
        if (dev != device) {
            // buffers of another device: release them once its work is done
            if (ws || norm) CHECK_HIP_EX(hipDeviceSynchronize());
            if (ws) CHECK_HIP_EX(hipFree(ws));
            if (norm) CHECK_HIP_EX(hipFree(norm));
            ws = nullptr;
            norm = nullptr;
            bytes = 0;
            device = dev;
        }
        if (!norm) CHECK_HIP_EX(hipMalloc(&norm, sizeof(float)));
        if (need > bytes) {
            if (ws) {
                CHECK_HIP_EX(hipStreamSynchronize(Hip::stream()));
                CHECK_HIP_EX(hipFree(ws));
                ws = nullptr;
            }
            CHECK_HIP_EX(hipMalloc(&ws, need));
            bytes = need;
        }
    }
};

NormScratch& scratch() {
    thread_local NormScratch s;
    return s;
}

struct FloatList {
    std::vector<float*> ptr;
    std::vector<int64_t> size;
};

FloatList list_of(const std::vector<tensor<float>*>& ts, const char* what) {
    FloatList l;
    l.ptr.reserve(ts.size());
    l.size.reserve(ts.size());
    for (size_t i = 0; i < ts.size(); ++i) {
        if (!ts[i]) throw std::invalid_argument(std::string(what) + ": null tensor in the list");
        l.ptr.push_back(ts[i]->data());
        l.size.push_back(ts[i]->size());
    }
    return l;
}

// The norm of `grads` into scratch().norm; with max_norm > 0 and clip set,
// the gradients are also scaled in place.
const float* device_norm(const std::vector<tensor<float>*>& grads, bool clip, float max_norm) {
    FloatList l = list_of(grads, "clip_grad_norm");
    const int count = (int)l.ptr.size();
    NormScratch& s = scratch();
    s.reserve(df_grad_norm_workspace_bytes(count, l.size.data()));
    if (clip)
        CHECK_DF_EX(df_clip_grad_norm_f32(l.ptr.data(), l.size.data(), count, max_norm, s.norm, s.ws, s.bytes,
                                          stream_arg()));
    else
        CHECK_DF_EX(df_grad_norm_f32(const_cast<const float* const*>(l.ptr.data()), l.size.data(), count, s.norm,
                                     s.ws, s.bytes, stream_arg()));
    return s.norm;
}

}  // namespace

namespace utils {
template <>
void clip_grad_norm<float>(std::vector<tensor<float>*>& gradients, float max_norm) {
    device_norm(gradients, true, max_norm);
}
}  // namespace utils

template <>
void AdamOptimizer<float>::update_parameters(const std::vector<tensor<float>*>& parameters,
                                             const std::vector<tensor<float>*>& gradients) {
    Optimizer<float>::update_parameters(parameters, gradients);
    for (auto* param : parameters) {
        if (m_.find(param) == m_.end()) {
            auto m_buf = std::make_unique<tensor<float>>(param->shape());
            auto v_buf = std::make_unique<tensor<float>>(param->shape());
            m_buf->fill(0.0f);
            v_buf->fill(0.0f);
            m_.emplace(param, std::move(m_buf));
            v_.emplace(param, std::move(v_buf));
        }
    }
}

template <>
void AdamOptimizer<float>::zero_grad() {
    for (auto* grad : this->gradients_) grad->fill(0.0f);
}

template <>
void AdamOptimizer<float>::launch(const float* clip_norm, float max_norm) {
    const auto& params = this->parameters_;
    const auto& grads = this->gradients_;
    if (grads.size() < params.size())
        throw std::invalid_argument("AdamOptimizer::step: fewer gradients than parameters");
    const size_t n = params.size();
    std::vector<float*> p(n), m(n), v(n);
    std::vector<const float*> g(n);
    std::vector<int64_t> sizes(n);
    for (size_t i = 0; i < n; ++i) {
        if (grads[i]->size() != params[i]->size())
            throw std::invalid_argument("AdamOptimizer::step: gradient " + std::to_string(i) +
                                        " differs in size from its parameter");
        p[i] = params[i]->data();
        g[i] = grads[i]->data();
        m[i] = m_.at(params[i])->data();
        v[i] = v_.at(params[i])->data();
        sizes[i] = params[i]->size();
    }
    CHECK_DF_EX(df_adam_update_f32(p.data(), g.data(), m.data(), v.data(), sizes.data(), (int)n, learning_rate_,
                                   beta1_, beta2_, epsilon_, weight_decay_, timestep_, clip_norm, max_norm,
                                   stream_arg()));
}

template <>
void AdamOptimizer<float>::step() {
    ++timestep_;
    launch(nullptr, 0.0f);
}

template <>
const float* AdamOptimizer<float>::step_clipped(float max_norm) {
    ++timestep_;
    const float* norm = device_norm(this->gradients_, false, max_norm);
    launch(norm, max_norm);
    return norm;
}

template class AdamOptimizer<float>;

}  // namespace dnn
