// FullyConnectedLayer<TT> in fp8 compute (the reference's
// dnn/layers/fully_connected_layer.cu:110-406), all device work through the
// C ABI on Hip::stream().
#include "dnn/layers/fully_connected_layer.hpp"

#include <algorithm>
#include <cmath>
#include <random>
#include <stdexcept>
#include <type_traits>
#include <vector>

#include "dnn/core/hip.hpp"
#include "dnn/utils/common.hpp"

namespace dnn {

namespace {
inline int round16(int v) { return (v + 15) & ~15; }
inline void* st() { return reinterpret_cast<void*>(Hip::stream()); }

// absmax (and, with scale_dev, the scale for fmt) of n elements of TT
template <typename TT>
void absmax_of(const TT* x, int64_t n, int fmt, float* absmax_dev, float* scale_dev, void* ws, size_t wb) {
    if constexpr (std::is_same_v<TT, float>) {
        CHECK_DF_EX(df_absmax_scale_f32(x, n, fmt, absmax_dev, scale_dev, ws, wb, st()));
    } else if constexpr (std::is_same_v<TT, __half>) {
        CHECK_DF_EX(df_absmax_scale_f16(reinterpret_cast<const uint16_t*>(x), n, fmt, absmax_dev, scale_dev, ws, wb,
                                        st()));
    } else {
        CHECK_DF_EX(df_absmax_scale_bf16(reinterpret_cast<const uint16_t*>(x), n, fmt, absmax_dev, scale_dev, ws, wb,
                                         st()));
    }
}
}  // namespace

template <typename TT>
FullyConnectedLayer<TT>::Scratch::~Scratch() {
    if (p) (void)hipFree(p);
}

template <typename TT>
uint8_t* FullyConnectedLayer<TT>::Scratch::get(size_t n, bool zeroed) {
    if (n == 0) n = 16;
    if (n > bytes) {
        if (p) {
            CHECK_HIP_EX(hipStreamSynchronize(Hip::stream()));  // previous users are done
            CHECK_HIP_EX(hipFree(p));
            p = nullptr;
        }
        const size_t alloc = (n + 255) & ~size_t(255);
        CHECK_HIP_EX(hipMalloc(&p, alloc));
        if (zeroed) CHECK_HIP_EX(hipMemset(p, 0, alloc));
        bytes = alloc;
    }
    return p;
}

template <typename TT>
FullyConnectedLayer<TT>::FullyConnectedLayer(int in_features, int out_features, bool training_enabled)
    : LayerWeightBias<TT>(tensor<TT>({out_features, in_features}), tensor<TT>({1, out_features, 1, 1}),
                          tensor<TT>({out_features, in_features}), tensor<TT>({1, out_features, 1, 1}),
                          training_enabled),
      in_features_(in_features),
      out_features_(out_features) {
    if (in_features <= 0 || out_features <= 0) throw std::invalid_argument("FullyConnectedLayer: bad sizes");
    initialize_weights();
}

// Xavier/Glorot uniform weights, zero bias (reference :359-385).
template <typename TT>
void FullyConnectedLayer<TT>::initialize_weights() {
    std::random_device rd;
    std::mt19937 gen(rd());
    const float limit = std::sqrt(6.0f / (in_features_ + out_features_));
    std::uniform_real_distribution<float> dist(-limit, limit);
    std::vector<TT> w(this->weights_.size());
    std::vector<TT> b(this->bias_.size());
    for (auto& v : w) v = static_cast<TT>(dist(gen));
    for (auto& v : b) v = static_cast<TT>(0.0f);
    this->weights_.upload(w.data());
    this->bias_.upload(b.data());
}

// absmax -> scale (written to scale_dev) -> 2-D codes (row copy q, transposed
// copy qt, optional fp32 column sums) in one stream-ordered call
// (df_quantize_2d_jit: the same results as the absmax call followed by the
// 2-D quantize, without the one-block launch between them).
template <typename TT>
void FullyConnectedLayer<TT>::quantize_operand(const TT* x, int rows, int cols, int fmt, float* scale_dev, uint8_t* q,
                                               int ldq, uint8_t* qt, int ldqt, float* colsum) {
    constexpr int dt = dtype_traits<TT>::value;
    const size_t wb = df_quantize_2d_jit_workspace_bytes(rows, cols, colsum ? 1 : 0);
    CHECK_DF_EX(df_quantize_2d_jit(dt, x, rows, cols, fmt, nullptr, scale_dev, q, ldq, qt, ldqt, colsum,
                                   colsum_ws_.get(wb), wb, st()));
}

template <typename TT>
void FullyConnectedLayer<TT>::set_delayed_scaling(int history_len) {
    if (history_len < 0 || history_len > 1024)
        throw std::invalid_argument("FullyConnectedLayer::set_delayed_scaling: history length must be in [0, 1024]");
    history_len_ = history_len;
    for (Delayed* d : {&dx_, &dw_, &ddy_}) {
        d->seeded = false;
        d->cur = 0;
        if (history_len > 0) {
            d->hist.get((size_t)history_len * sizeof(float));
            d->scales.get(3 * sizeof(float));
        }
    }
    sx_used_ = sw_used_ = nullptr;
}

template <typename TT>
const float* FullyConnectedLayer<TT>::amax_history(int operand) {
    if (history_len_ == 0 || operand < 0 || operand > 2)
        throw std::invalid_argument("FullyConnectedLayer::amax_history: no such history");
    Delayed* d = operand == 0 ? &dx_ : operand == 1 ? &dw_ : &ddy_;
    return reinterpret_cast<const float*>(d->hist.p);
}

template <typename TT>
const float* FullyConnectedLayer<TT>::quantize_delayed(Delayed& d, const TT* x, int rows, int cols, int fmt,
                                                       uint8_t* q, int ldq, uint8_t* qt, int ldqt, float* colsum) {
    constexpr int dt = dtype_traits<TT>::value;
    float* hist = reinterpret_cast<float*>(d.hist.get((size_t)history_len_ * sizeof(float)));
    float* sc = reinterpret_cast<float*>(d.scales.get(3 * sizeof(float)));
    float* used = sc + d.cur;
    float* next = sc + (d.cur ^ 1);
    if (!d.seeded) {
        // the first pass seeds the history with its own absmax
        const size_t ab = df_absmax_workspace_bytes();
        uint8_t* aws = absmax_ws_.get(ab);
        absmax_of(x, (int64_t)rows * cols, fmt, sc + 2, nullptr, aws, ab);
        CHECK_DF_EX(df_amax_history_init(sc + 2, fmt, hist, history_len_, used, st()));
        d.seeded = true;
    }
    const size_t wb = df_quantize_2d_delayed_workspace_bytes(rows, cols, q ? ldq : 0, qt ? ldqt : 0, colsum ? 1 : 0);
    CHECK_DF_EX(df_quantize_2d_delayed(dt, x, rows, cols, cols, fmt, used, next, hist, history_len_, q, ldq, qt, ldqt,
                                       colsum, colsum_ws_.get(wb), wb, st()));
    d.cur ^= 1;
    return used;
}

template <typename TT>
const float* FullyConnectedLayer<TT>::quantize_input(const tensor<TT>& input, int N, const LayerNormLayer<TT>* norm,
                                                     uint8_t* xq, int Kp, uint8_t* xt, int Np, float* jit_scale) {
    constexpr int dt = dtype_traits<TT>::value;
    if (!norm) {
        if (history_len_ > 0)
            return quantize_delayed(dx_, input.data(), N, in_features_, DF_FMT_E4M3, xq, Kp, xt, Np, nullptr);
        quantize_operand(input.data(), N, in_features_, DF_FMT_E4M3, jit_scale, xq, Kp, xt, Np, nullptr);
        return jit_scale;
    }
    // LayerNorm fused into the quantize: statistics pass, then codes
    const size_t wb = df_layernorm_workspace_bytes(N, in_features_, Kp, xt ? Np : 0);
    void* ws = colsum_ws_.get(wb);
    const void* g = norm->affine() ? norm->gamma().data() : nullptr;
    const void* b = norm->affine() ? norm->beta().data() : nullptr;
    const float eps = norm->epsilon();
    if (history_len_ == 0) {
        CHECK_DF_EX(df_layernorm_quantize(dt, input.data(), N, in_features_, in_features_, g, b, eps, nullptr, 0,
                                          DF_FMT_E4M3, jit_scale, nullptr, xq, Kp, xt, Np, ws, wb, st()));
        return jit_scale;
    }
    Delayed& d = dx_;
    float* hist = reinterpret_cast<float*>(d.hist.get((size_t)history_len_ * sizeof(float)));
    float* sc = reinterpret_cast<float*>(d.scales.get(3 * sizeof(float)));
    float* used = sc + d.cur;
    float* next = sc + (d.cur ^ 1);
    if (!d.seeded) {
        // the first pass runs at its own absmax, which seeds the history
        CHECK_DF_EX(df_layernorm_quantize(dt, input.data(), N, in_features_, in_features_, g, b, eps, nullptr, 0,
                                          DF_FMT_E4M3, used, sc + 2, xq, Kp, xt, Np, ws, wb, st()));
        CHECK_DF_EX(df_amax_history_init(sc + 2, DF_FMT_E4M3, hist, history_len_, next, st()));
        d.seeded = true;
    } else {
        CHECK_DF_EX(df_layernorm_quantize_delayed(dt, input.data(), N, in_features_, in_features_, g, b, eps, nullptr,
                                                  0, DF_FMT_E4M3, used, next, hist, history_len_, xq, Kp, xt, Np, ws,
                                                  wb, st()));
    }
    d.cur ^= 1;
    return used;
}

template <typename TT>
tensor<TT> FullyConnectedLayer<TT>::forward(const tensor<TT>& input) {
    return forward_impl(input, nullptr);
}

template <typename TT>
tensor<TT> FullyConnectedLayer<TT>::forward(const tensor<TT>& input, LayerNormLayer<TT>& norm) {
    if (norm.norm_size() != in_features_)
        throw std::invalid_argument("FullyConnectedLayer::forward: LayerNorm over " + std::to_string(norm.norm_size()) +
                                    " values feeds a layer of " + std::to_string(in_features_) + " inputs");
    norm.rows_of(input);  // throws on a ragged input
    norm.note_input(input);
    return forward_impl(input, &norm);
}

template <typename TT>
float* FullyConnectedLayer<TT>::input_scale_slot(int N) {
    if (!this->training_enabled_) return reinterpret_cast<float*>(scales_.get(4 * sizeof(float)));
    const std::vector<int> xt_shape{in_features_, round16(N)};
    if (!xt_cache_ || xt_cache_->shape() != xt_shape) xt_cache_.emplace(xt_shape);
    return xt_cache_->scale_data();
}

template <typename TT>
float* FullyConnectedLayer<TT>::grad_scale_slot() {
    return reinterpret_cast<float*>(scales_.get(4 * sizeof(float))) + 2;
}

template <typename TT>
tensor<TT> FullyConnectedLayer<TT>::forward(FullyConnectedLayer<TT>& prev, const tensor<TT>& input) {
    if (prev.out_features_ != in_features_)
        throw std::invalid_argument("FullyConnectedLayer::forward: a layer of " + std::to_string(prev.out_features_) +
                                    " outputs feeds a layer of " + std::to_string(in_features_) + " inputs");
    if (history_len_ > 0 || &prev == this) return forward(prev.forward(input));
    const auto& sh = input.shape();
    // checked before input_scale_slot may replace this layer's cached X^T
    if (sh.size() != 2 || sh[1] != prev.in_features_)
        throw std::invalid_argument("FullyConnectedLayer::forward: input must be [N, " +
                                    std::to_string(prev.in_features_) + "], got " + input.to_string());
    const int N = sh[0];
    cached_n_ = -1;  // until this forward completes, backward has no input to use
    float* slot = input_scale_slot(N);
    const tensor<TT> hidden = prev.forward_impl(input, nullptr, nullptr, slot);
    return forward_impl(hidden, nullptr, slot);
}

template <typename TT>
tensor<TT> FullyConnectedLayer<TT>::forward_impl(const tensor<TT>& input, LayerNormLayer<TT>* norm,
                                                 const float* in_scale, float* out_scale) {
    const auto& sh = input.shape();
    int N;
    if (norm) {
        N = norm->rows_of(input);  // any rank: runs of in_features values
    } else {
        if (sh.size() != 2 || sh[1] != in_features_)
            throw std::invalid_argument("FullyConnectedLayer::forward: input must be [N, " +
                                        std::to_string(in_features_) + "], got " + input.to_string());
        N = sh[0];
    }
    // A forward that throws past this point may have replaced the cached X^T
    // (another N) or overwritten its codes: backward then refuses rather than
    // reading it at the old N.
    cached_n_ = -1;
    tensor<TT> output({N, out_features_});
    if (N == 0) {  // an empty batch: its backward has zero weight and bias gradients
        cached_n_ = this->training_enabled_ ? 0 : -1;
        return output;
    }
    constexpr int dt = dtype_traits<TT>::value;
    const int Kp = round16(in_features_), Np = round16(N);
    float* sc = reinterpret_cast<float*>(scales_.get(4 * sizeof(float)));
    uint8_t* xq = codes_a_.get((size_t)N * Kp);
    uint8_t* xt = nullptr;
    float* sx_jit = sc;
    if (this->training_enabled_) {
        const std::vector<int> xt_shape{in_features_, Np};
        if (!xt_cache_ || xt_cache_->shape() != xt_shape) xt_cache_.emplace(xt_shape);
        xt = reinterpret_cast<uint8_t*>(xt_cache_->data());
        sx_jit = xt_cache_->scale_data();
    }
    const float* sx = sx_jit;
    if (in_scale) {  // the producer of `input` wrote its scale into sx_jit
        if (in_scale != sx_jit) throw std::logic_error("FullyConnectedLayer: input scale outside its slot");
        CHECK_DF_EX(df_quantize_2d(dt, input.data(), N, in_features_, in_features_, DF_FMT_E4M3, in_scale, xq, Kp, xt,
                                   xt ? Np : 0, st()));
    } else {
        sx = quantize_input(input, N, norm, xq, Kp, xt, Np, sx_jit);
    }
    uint8_t* wq = codes_b_.get((size_t)out_features_ * Kp);
    // in training, the same pass also writes W's transposed codes for the
    // backward's dX GEMM (the weights cannot change before the backward that
    // follows): one read of W per step instead of two, and no second absmax
    const int Op = round16(out_features_);
    uint8_t* wt = this->training_enabled_ ? codes_wt_.get((size_t)in_features_ * Op) : nullptr;
    const float* sw = sc + 1;
    if (history_len_ > 0) {
        sw = quantize_delayed(dw_, this->weights_.data(), out_features_, in_features_, DF_FMT_E4M3, wq, Kp, wt,
                              wt ? Op : 0, nullptr);
        sx_used_ = sx;
        sw_used_ = sw;
    } else {
        quantize_operand(this->weights_.data(), out_features_, in_features_, DF_FMT_E4M3, sc + 1, wq, Kp, wt,
                         wt ? Op : 0, nullptr);
        sx_used_ = sw_used_ = nullptr;
    }
    // a training forward has just written W^T codes of the current weights
    // (at the scale sw), so a load() before it no longer leaves them stale
    if (wt) wt_stale_ = false;
    if (out_scale) {
        const size_t gb = df_fp8_gemm_fwd_absmax_workspace_bytes(N, out_features_, in_features_);
        CHECK_DF_EX(df_fp8_gemm_fwd_absmax(xq, Kp, wq, Kp, N, out_features_, in_features_, sx, sw, dt,
                                           this->bias_.data(), dt, output.data(), out_features_, DF_FMT_E4M3, nullptr,
                                           out_scale, gemm_ws_.get(gb), gb, st()));
    } else {
        const size_t gb = df_fp8_gemm_workspace_bytes(N, out_features_, in_features_);
        CHECK_DF_EX(df_fp8_gemm_fwd(xq, Kp, wq, Kp, N, out_features_, in_features_, sx, sw, dt, this->bias_.data(),
                                    dt, output.data(), out_features_, gemm_ws_.get(gb), gb, st()));
    }
    cached_n_ = this->training_enabled_ ? N : -1;
    return output;
}

template <typename TT>
tensor<TT> FullyConnectedLayer<TT>::backward(const tensor<TT>& grad_output) {
    return backward_impl(grad_output);
}

template <typename TT>
tensor<TT> FullyConnectedLayer<TT>::backward(FullyConnectedLayer<TT>& next, const tensor<TT>& grad_output) {
    if (next.in_features_ != out_features_)
        throw std::invalid_argument("FullyConnectedLayer::backward: a layer of " + std::to_string(out_features_) +
                                    " outputs feeds a layer of " + std::to_string(next.in_features_) + " inputs");
    if (history_len_ > 0 || &next == this) return backward(next.backward(grad_output));
    float* slot = grad_scale_slot();
    const tensor<TT> grad_hidden = next.backward_impl(grad_output, nullptr, slot);
    return backward_impl(grad_hidden, slot);
}

template <typename TT>
tensor<TT> FullyConnectedLayer<TT>::backward_impl(const tensor<TT>& grad_output, const float* dy_scale,
                                                  float* dx_scale) {
    if (!this->training_enabled_)
        throw std::runtime_error("FullyConnectedLayer: backward called without input argument in stateless mode");
    if (cached_n_ < 0 || (cached_n_ > 0 && !xt_cache_))
        throw std::runtime_error("FullyConnectedLayer: input_cache_ not set for backward");
    const int N = cached_n_;
    const auto& sh = grad_output.shape();
    if (sh.size() != 2 || sh[0] != N || sh[1] != out_features_)
        throw std::invalid_argument("FullyConnectedLayer::backward: grad_output must be [" + std::to_string(N) + ", " +
                                    std::to_string(out_features_) + "], got " + grad_output.to_string());
    if (N == 0) {  // sums over no rows; dx_scale stays unwritten, as no empty dX is quantized
        this->grad_weights_.zero();
        this->grad_bias_.zero();
        return tensor<TT>({0, in_features_});
    }
    constexpr int dt = dtype_traits<TT>::value;
    const int Np = round16(N), Op = round16(out_features_);
    float* sc = reinterpret_cast<float*>(scales_.get(4 * sizeof(float)));
    // dY -> e5m2 row copy (for dX), transposed copy (for dW), and db
    uint8_t* dyq = codes_a_.get((size_t)N * Op);
    uint8_t* dyt = codes_c_.get((size_t)out_features_ * Np);
    float* db = reinterpret_cast<float*>(colsum_.get((size_t)out_features_ * sizeof(float)));
    // W^T codes and their scale: written by the forward's W pass, or here
    // when load() replaced the weights after that forward (the reference's
    // backward reads weights_ as they are now)
    const uint8_t* wt = codes_wt_.p;
    const float* sdy = sc + 2;
    const float* sw = sc + 1;
    const float* sx = xt_cache_->scale_data();
    if (wt_stale_) {
        uint8_t* wtn = codes_wt_.get((size_t)in_features_ * Op);
        quantize_operand(this->weights_.data(), out_features_, in_features_, DF_FMT_E4M3, sc + 1, nullptr, 0, wtn,
                         Op, nullptr);
        wt = wtn;
        wt_stale_ = false;
        sw_used_ = nullptr;  // these codes are at the just-in-time scale sc + 1
    }
    if (dy_scale) {  // the layer this one feeds wrote grad_output's scale into sc + 2
        if (dy_scale != sc + 2) throw std::logic_error("FullyConnectedLayer: gradient scale outside its slot");
        const size_t cb = df_quantize_2d_workspace_bytes(N, out_features_);
        CHECK_DF_EX(df_quantize_2d_colsum(dt, grad_output.data(), N, out_features_, out_features_, DF_FMT_E5M2,
                                          dy_scale, dyq, Op, dyt, Np, db, colsum_ws_.get(cb), cb, st()));
    } else if (history_len_ > 0 && sx_used_) {
        sdy = quantize_delayed(ddy_, grad_output.data(), N, out_features_, DF_FMT_E5M2, dyq, Op, dyt, Np, db);
        if (sw_used_) sw = sw_used_;
        sx = sx_used_;
    } else {
        quantize_operand(grad_output.data(), N, out_features_, DF_FMT_E5M2, sc + 2, dyq, Op, dyt, Np, db);
    }
    tensor<TT> grad_input({N, in_features_});
    // dX (fc_backward_input) and dW (fc_backward_weights) in one launch
    const uint8_t* xtc = reinterpret_cast<const uint8_t*>(xt_cache_->data());
    if (dx_scale) {
        const size_t gb = df_fp8_gemm_bwd_absmax_workspace_bytes(N, out_features_, in_features_);
        CHECK_DF_EX(df_fp8_gemm_bwd_absmax(dyq, Op, wt, Op, dyt, Np, xtc, Np, N, out_features_, in_features_, sdy, sw,
                                           sx, dt, grad_input.data(), in_features_, dt, this->grad_weights_.data(),
                                           in_features_, DF_FMT_E5M2, nullptr, dx_scale, gemm_ws_.get(gb), gb,
                                           st()));
    } else {
        const size_t gb = df_fp8_gemm_bwd_workspace_bytes(N, out_features_, in_features_);
        CHECK_DF_EX(df_fp8_gemm_bwd(dyq, Op, wt, Op, dyt, Np, xtc, Np, N, out_features_, in_features_, sdy, sw, sx, dt,
                                    grad_input.data(), in_features_, dt, this->grad_weights_.data(), in_features_,
                                    gemm_ws_.get(gb), gb, st()));
    }
    CHECK_DF_EX(df_convert(DF_DTYPE_FLOAT32, db, dt, this->grad_bias_.data(), out_features_, st()));
    return grad_input;
}

template <typename TT>
void FullyConnectedLayer<TT>::save(std::ostream& out) const {
    out.write(reinterpret_cast<const char*>(&in_features_), sizeof(in_features_));
    out.write(reinterpret_cast<const char*>(&out_features_), sizeof(out_features_));
    this->weights_.save(out);
    this->bias_.save(out);
}

template <typename TT>
void FullyConnectedLayer<TT>::save_fp8(std::ostream& out) const {
    out.write(reinterpret_cast<const char*>(&in_features_), sizeof(in_features_));
    out.write(reinterpret_cast<const char*>(&out_features_), sizeof(out_features_));
    quantize<fp8_e4m3>(this->weights_).save(out);
    this->bias_.save(out);
}

template <typename TT>
void FullyConnectedLayer<TT>::load(std::istream& in) {
    const int old_in = in_features_, old_out = out_features_;
    in.read(reinterpret_cast<char*>(&in_features_), sizeof(in_features_));
    in.read(reinterpret_cast<char*>(&out_features_), sizeof(out_features_));
    this->weights_.load(in);
    this->bias_.load(in);
    if (this->grad_weights_.shape() != this->weights_.shape())
        this->grad_weights_ = tensor<TT>(this->weights_.shape());
    if (this->grad_bias_.shape() != this->bias_.shape()) this->grad_bias_ = tensor<TT>(this->bias_.shape());
    if (in_features_ != old_in || out_features_ != old_out) {
        // a layer of another shape: the cached input no longer fits
        xt_cache_.reset();
        cached_n_ = -1;
    }
    // like the reference, a backward after load() uses the cached input and
    // the loaded weights: their W^T codes are made again by that backward
    wt_stale_ = true;
    sw_used_ = nullptr;
}

template class FullyConnectedLayer<float>;
template class FullyConnectedLayer<__half>;
template class FullyConnectedLayer<bfloat16>;

}  // namespace dnn
