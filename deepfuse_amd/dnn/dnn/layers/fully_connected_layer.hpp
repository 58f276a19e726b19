// dnn/layers/fully_connected_layer.hpp -- the fp8 Linear layer (drop-in).
//
// Public contract of the reference's FullyConnectedLayer<TT>
// (dnn/layers/fully_connected_layer.cuh:21-52, .cu:111-402): W is
// [out, in], bias [1, out, 1, 1], input [N, in] -> output [N, out];
// forward caches what backward needs when training is enabled; backward
// returns dX [N, in] and overwrites grad_weights [out, in] and grad_bias;
// backward without training (or before a forward) throws; save/load write
// in, out, weights, bias.
//
// Compute is fp8 on CDNA4 MFMA through the C ABI: forward quantizes X and
// W to e4m3 (per-tensor absmax scales) and runs Y = Xq . Wq^T * sx * sw + b;
// backward quantizes dY to e5m2 (its column sums give grad_bias in the same
// pass), dX = dYq . W * sdy * sw, dW = dYq^T . X * sdy * sx, all with fp32
// accumulation.  Instead of a full clone of the input, training caches the
// transposed e4m3 codes of X (one byte per element) and their scale, and the
// forward's pass over W also writes W's transposed codes for the backward:
// backward uses the weights its forward used (the reference re-reads
// weights_, which is the same unless they are changed in between).
// TT: float or bfloat16.
#pragma once

#include <iostream>
#include <optional>
#include <string>
#include <type_traits>

#include "dnn/core/layer.hpp"
#include "dnn/layers/layer_norm_layer.hpp"
#include "dnn/core/tensor.hpp"

namespace dnn {

template <typename TT>
class FullyConnectedLayer : public LayerWeightBias<TT> {
public:
    FullyConnectedLayer(int in_features, int out_features, bool training_enabled = false);
    ~FullyConnectedLayer() override = default;

    tensor<TT> forward(const tensor<TT>& input) override;
    // forward(norm.forward(input)) with the LayerNorm fused into the
    // quantize of this layer's input: the normalised tensor is never
    // written; the codes (and the cached transposed codes for backward) come
    // straight from `input` (df_layernorm_quantize).  Same values as the
    // unfused pair.  norm records its input for its own backward as
    // norm.forward would.
    tensor<TT> forward(const tensor<TT>& input, LayerNormLayer<TT>& norm);
    // forward(prev.forward(input)) where prev's output feeds this layer with
    // nothing in between (the reference block's fc1 -> fc2,
    // transformer_block.cu:79-81): prev's GEMM also gives the absmax of its
    // output (df_fp8_gemm_fwd_absmax), which sets this layer's input scale,
    // so the output is not read again for it.  Same values as the unfused
    // pair; prev caches for its backward as prev.forward would.  With
    // delayed scaling on this layer it is the unfused pair.
    tensor<TT> forward(FullyConnectedLayer<TT>& prev, const tensor<TT>& input);
    tensor<TT> backward(const tensor<TT>& grad_output) override;
    // backward(next.backward(grad_output)) where next is the layer this one
    // feeds (transformer_block.cu:127-134): next's backward GEMM also gives
    // the absmax of its input gradient (df_fp8_gemm_bwd_absmax), this
    // layer's output gradient, which sets its dY scale.  Same values as the
    // unfused pair, and the same fallback.
    tensor<TT> backward(FullyConnectedLayer<TT>& next, const tensor<TT>& grad_output);

    std::string name() const override { return "FullyConnected"; }
    void initialize_weights() override;
    void save(std::ostream& out) const override;
    void load(std::istream& in) override;
    // The reference's layout (in, out, weights, bias; fully_connected_layer.cu:
    // 388-402) with the weights as an fp8 e4m3 record (codes + scale, a
    // quarter of the fp32 bytes).  load() reads both forms; the fp8 form
    // comes back as the dequantized weights.
    void save_fp8(std::ostream& out) const;

    // Delayed scaling (an addition: the reference has no quantizer).  With
    // history_len in [1, 1024] the scales of X, W and dY come from amax
    // histories of their last history_len passes instead of an absmax pass
    // over the current data; each pass measures its own absmax on the way
    // and pushes it.  The first pass of each operand seeds its history with
    // its own absmax, so it equals the just-in-time pass.  Values beyond the
    // inherited range saturate.  0 (the default) is the just-in-time path.
    void set_delayed_scaling(int history_len);
    int delayed_scaling() const { return history_len_; }
    // device pointer to an operand's history (0: X, 1: W, 2: dY)
    const float* amax_history(int operand);

private:
    // device scratch reused across calls, grown on demand
    struct Scratch {
        uint8_t* p = nullptr;
        size_t bytes = 0;
        ~Scratch();
        uint8_t* get(size_t n, bool zeroed = false);
    };
    void quantize_operand(const TT* x, int rows, int cols, int fmt, float* scale_dev, uint8_t* q, int ldq,
                          uint8_t* qt, int ldqt, float* colsum);
    // delayed-scaling state of one operand: history, two scale slots used in
    // turn (the codes' scale stays valid until the pass after next), one
    // absmax slot for seeding
    struct Delayed {
        Scratch hist, scales;
        int cur = 0;
        bool seeded = false;
    };
    // quantizes with the operand's current scale, pushes this pass's absmax;
    // returns the device pointer of the scale the codes were made with
    const float* quantize_delayed(Delayed& d, const TT* x, int rows, int cols, int fmt, uint8_t* q, int ldq,
                                  uint8_t* qt, int ldqt, float* colsum);
    // input operand codes: from `input` itself, or from LayerNorm(input)
    // when norm is given; returns the device pointer of their scale
    const float* quantize_input(const tensor<TT>& input, int N, const LayerNormLayer<TT>* norm, uint8_t* xq, int Kp,
                                uint8_t* xt, int Np, float* jit_scale);
    // in_scale: the input's scale is already in input_scale_slot(N) (written
    // by the layer that produced the input); out_scale: the GEMM also writes
    // the e4m3 scale of the output there, for the layer it feeds
    tensor<TT> forward_impl(const tensor<TT>& input, LayerNormLayer<TT>* norm, const float* in_scale = nullptr,
                            float* out_scale = nullptr);
    // dy_scale: grad_output's e5m2 scale is already there; dx_scale: the
    // backward GEMM also writes the e5m2 scale of the input gradient there
    tensor<TT> backward_impl(const tensor<TT>& grad_output, const float* dy_scale = nullptr,
                             float* dx_scale = nullptr);
    // where the scale of an N-row input's codes lives (beside the cached X^T
    // codes when training)
    float* input_scale_slot(int N);
    // where grad_output's scale lives
    float* grad_scale_slot();

    int in_features_;
    int out_features_;
    int cached_n_ = -1;                        // tokens of the cached forward
    std::optional<tensor<fp8_e4m3>> xt_cache_;  // X^T codes [in, round16(N)] + scale
    Scratch absmax_ws_, colsum_ws_, gemm_ws_, codes_a_, codes_b_, codes_c_, scales_, colsum_;
    Scratch codes_wt_;  // W^T codes [in, round16(out)] from the training forward, read by backward
    bool wt_stale_ = false;  // load() replaced the weights after the forward that wrote codes_wt_
    int history_len_ = 0;
    Delayed dx_, dw_, ddy_;
    const float* sx_used_ = nullptr;  // delayed: scales of the cached forward's X and W codes
    const float* sw_used_ = nullptr;
};

}  // namespace dnn
