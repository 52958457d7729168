// layer.cpp -- the drop-in modules (reference core/layer.cpp).
//
// LayerNorm, BatchNorm2d and MultiHeadAttention call include/wm_layers.h
// (forward and backward closure on the device); Dropout draws its mask on the
// device; the activations, Softmax / LogSoftmax, Flatten, Linear, the
// convolutions and the pools are the reference's Tensor-op compositions (the
// convolutions and pools reach Tensor ops this build does not provide and
// throw there).  Embedding, LSTM and GRU construct and count their parameters
// as the reference does and throw from forward().  Summaries and parameter
// counting are host bookkeeping, as in the reference.
#include "layer.h"

#include <cmath>
#include <cstdint>
#include <cstdio>
#include <memory>
#include <random>
#include <stdexcept>
#include <string>

#include "wm_hip.h"
#include "wm_gemm.h"
#include "wm_layers.h"

namespace {

void ck(int rc, const char* what) {
    if (rc != WM_OK) throw std::runtime_error(std::string("whitematter_amd ") + what + ": " + wm_last_error());
}

[[noreturn]] void out_of_scope(const char* what) {
    throw std::logic_error(std::string(what) + ": not part of the MI355X elementwise/broadcast/reduction build");
}

// The generator every constructor draws its initial weights from, seeded as
// the reference's file-scope std::mt19937 (core/layer.cpp:5), so the same
// construction sequence gives the same weights.
std::mt19937& init_rng() {
    static std::mt19937 rng(123);
    return rng;
}

// A parameter of `shape` filled element by element from `dist`, in storage
// order (the reference's range-for over weight->data).
TensorPtr drawn(const std::vector<size_t>& shape, float stddev) {
    std::normal_distribution<float> dist(0.0f, stddev);
    size_t n = 1;
    for (auto d : shape) n *= d;
    std::vector<float> v(n);
    for (auto& x : v) x = dist(init_rng());
    return Tensor::create(v, shape, true);
}

// A gradient buffer sized like the tensor's data.
float* grad_target(const TensorPtr& t, int* accumulate) {
    if (t->grad.size() != t->data.size()) t->grad = wm::DeviceVector(t->data.size());
    return t->grad.dev_accum(accumulate);
}

std::string with_commas(size_t n) {
    std::string s = std::to_string(n);
    for (int pos = (int)s.size() - 3; pos > 0; pos -= 3) s.insert((size_t)pos, ",");
    return s;
}

std::string shape_str(const std::vector<size_t>& shape) {
    if (shape.empty()) return "-";
    std::string s = "[";
    for (size_t i = 0; i < shape.size(); ++i) s += (i ? ", " : "") + std::to_string(shape[i]);
    return s + "]";
}

// Position in the counter-based dropout stream: advanced by each mask's size.
uint64_t& dropout_counter() {
    static uint64_t c = 123;
    return c;
}

}  // namespace

// ---- Module ----------------------------------------------------------------

size_t Module::num_parameters() const {
    size_t total = 0;
    for (const auto& p : const_cast<Module*>(this)->parameters()) total += p->size();
    return total;
}

size_t Module::num_trainable_parameters() const {
    size_t total = 0;
    for (const auto& p : const_cast<Module*>(this)->parameters())
        if (p->requires_grad) total += p->size();
    return total;
}

// ---- Tensor-op modules (core/layer.cpp:7-45, :398 Flatten) ----------------------

Linear::Linear(size_t in_features, size_t out_features) : in_features(in_features), out_features(out_features) {
    weight = Tensor::xavier(in_features, out_features, true);
    bias = Tensor::zeros({out_features}, true);
}

TensorPtr Linear::forward(const TensorPtr& input) { return input->matmul(weight)->add(bias); }
std::vector<TensorPtr> Linear::parameters() { return {weight, bias}; }

TensorPtr ReLU::forward(const TensorPtr& input) { return input->relu(); }
TensorPtr Sigmoid::forward(const TensorPtr& input) { return input->sigmoid(); }
TensorPtr Tanh::forward(const TensorPtr& input) { return input->tanh_(); }

Softmax::Softmax(int dim) : dim(dim) {}
TensorPtr Softmax::forward(const TensorPtr& input) { return input->softmax(dim); }

LogSoftmax::LogSoftmax(int dim) : dim(dim) {}
TensorPtr LogSoftmax::forward(const TensorPtr& input) { return input->log_softmax(dim); }

TensorPtr Flatten::forward(const TensorPtr& input) { return input->flatten(1); }

// ---- Dropout (core/layer.cpp:45-73) ---------------------------------------------

Dropout::Dropout(float p) : p(p), training(true) {}

// Training: input * mask, mask_i in {0, 1/(1-p)} drawn on the device; the
// product's closure gives the reference's input->grad += grad * mask.
TensorPtr Dropout::forward(const TensorPtr& input) {
    if (!training || p == 0.0f) return input;
    const int64_t n = (int64_t)input->data.size();
    auto mask = Tensor::create(input->shape, false);
    ck(wm_dropout_mask(mask->data.dev_write(), n, p, dropout_counter()), "Dropout");
    dropout_counter() += (uint64_t)n;
    return input->mul(mask);
}

// ---- convolutions and pools (core/layer.cpp:100-192) ----------------------------

Conv2d::Conv2d(size_t in_channels, size_t out_channels, size_t kernel_size, size_t stride, size_t padding)
    : in_channels(in_channels), out_channels(out_channels), kernel_size(kernel_size), stride(stride),
      padding(padding) {
    weight = drawn({out_channels, in_channels, kernel_size, kernel_size},
                   std::sqrt(2.0f / (in_channels * kernel_size * kernel_size)));
    bias = Tensor::zeros({out_channels}, true);
}

TensorPtr Conv2d::forward(const TensorPtr& input) { return input->conv2d(weight, bias, stride, padding); }
std::vector<TensorPtr> Conv2d::parameters() { return {weight, bias}; }

ConvTranspose2d::ConvTranspose2d(size_t in_channels, size_t out_channels, size_t kernel_size, size_t stride,
                                 size_t padding, size_t output_padding)
    : in_channels(in_channels), out_channels(out_channels), kernel_size(kernel_size), stride(stride),
      padding(padding), output_padding(output_padding) {
    weight = drawn({in_channels, out_channels, kernel_size, kernel_size},
                   std::sqrt(2.0f / (in_channels * kernel_size * kernel_size)));
    bias = Tensor::zeros({out_channels}, true);
}

TensorPtr ConvTranspose2d::forward(const TensorPtr& input) {
    return input->conv_transpose2d(weight, bias, stride, padding, output_padding);
}
std::vector<TensorPtr> ConvTranspose2d::parameters() { return {weight, bias}; }

MaxPool2d::MaxPool2d(size_t kernel_size, size_t stride)
    : kernel_size(kernel_size), stride(stride == 0 ? kernel_size : stride) {}
TensorPtr MaxPool2d::forward(const TensorPtr& input) { return input->maxpool2d(kernel_size, stride); }

AvgPool2d::AvgPool2d(size_t kernel_size, size_t stride)
    : kernel_size(kernel_size), stride(stride == 0 ? kernel_size : stride) {}
TensorPtr AvgPool2d::forward(const TensorPtr& input) { return input->avgpool2d(kernel_size, stride); }

// ---- BatchNorm2d (core/layer.cpp:194-380) -----------------------------------------

BatchNorm2d::BatchNorm2d(size_t num_features, float eps, float momentum)
    : num_features(num_features), eps(eps), momentum(momentum), training(true) {
    gamma = Tensor::ones({num_features}, true);
    beta = Tensor::zeros({num_features}, true);
    running_mean = Tensor::zeros({num_features}, false);
    running_var = Tensor::ones({num_features}, false);
}

// Tracking follows the input only (core/layer.cpp:214): an input without
// requires_grad gives no closure, so gamma and beta get no gradient either.
TensorPtr BatchNorm2d::forward(const TensorPtr& input) {
    if (input->shape.size() != 4 || input->shape[1] != num_features)
        throw std::invalid_argument("BatchNorm2d: input must be [batch, num_features, height, width]");
    const int64_t B = (int64_t)input->shape[0], C = (int64_t)input->shape[1];
    const int64_t S = (int64_t)(input->shape[2] * input->shape[3]);
    const bool track = input->requires_grad && GradMode::is_enabled();
    auto result = Tensor::create(input->shape, track);
    auto mean = std::make_shared<wm::DeviceVector>((size_t)C);
    auto inv = std::make_shared<wm::DeviceVector>((size_t)C);
    ck(wm_batchnorm2d_fwd(input->data.dev(), gamma->data.dev(), beta->data.dev(), running_mean->data.dev_rw(),
                          running_var->data.dev_rw(), B, C, S, eps, momentum, training ? 1 : 0,
                          result->data.dev_write(), mean->dev_write(), inv->dev_write()),
       "BatchNorm2d");
    if (track) {
        auto in = input;
        auto gm = gamma;
        auto bt = beta;
        Tensor* res = result.get();
        result->parents = {in, gm, bt};
        result->grad_fn = [in, gm, bt, res, mean, inv, B, C, S]() {
            int ax = 0, ag = 0, ab = 0;
            float* gx = in->requires_grad ? grad_target(in, &ax) : nullptr;
            float* dg = gm->requires_grad ? grad_target(gm, &ag) : nullptr;
            float* db = bt->requires_grad ? grad_target(bt, &ab) : nullptr;
            ck(wm_batchnorm2d_bwd(res->grad.dev(), in->data.dev(), gm->data.dev(), mean->dev(), inv->dev(), B, C, S,
                                  gx, ax, dg, ag, db, ab),
               "BatchNorm2d backward");
        };
    }
    return result;
}

std::vector<TensorPtr> BatchNorm2d::parameters() { return {gamma, beta}; }

// ---- LayerNorm (core/layer.cpp:382-510) ---------------------------------------------

LayerNorm::LayerNorm(std::vector<size_t> normalized_shape, float eps) : normalized_shape(normalized_shape), eps(eps) {
    size_t size = 1;
    for (auto s : normalized_shape) size *= s;
    gamma = Tensor::ones({size}, true);
    beta = Tensor::zeros({size}, true);
}

LayerNorm::LayerNorm(size_t dim, float eps) : LayerNorm(std::vector<size_t>{dim}, eps) {}

TensorPtr LayerNorm::forward(const TensorPtr& input) {
    const size_t nd = normalized_shape.size();
    if (input->shape.size() < nd) throw std::invalid_argument("LayerNorm: input has fewer dims than normalized_shape");
    size_t n = 1, rows = 1;
    for (size_t i = 0; i < nd; ++i) {
        if (input->shape[input->shape.size() - nd + i] != normalized_shape[i])
            throw std::invalid_argument("LayerNorm: trailing dims do not match normalized_shape");
        n *= normalized_shape[i];
    }
    for (size_t i = 0; i + nd < input->shape.size(); ++i) rows *= input->shape[i];
    const bool track = input->requires_grad && GradMode::is_enabled();
    auto result = Tensor::create(input->shape, track);
    auto mean = std::make_shared<wm::DeviceVector>(rows);
    auto inv = std::make_shared<wm::DeviceVector>(rows);
    ck(wm_layernorm_fwd(input->data.dev(), gamma->data.dev(), beta->data.dev(), (int64_t)rows, (int64_t)n, eps,
                        result->data.dev_write(), mean->dev_write(), inv->dev_write()),
       "LayerNorm");
    if (track) {
        auto in = input;
        auto gm = gamma;
        auto bt = beta;
        Tensor* res = result.get();
        result->parents = {in, gm, bt};
        result->grad_fn = [in, gm, bt, res, mean, inv, rows, n]() {
            int ax = 0, ag = 0, ab = 0;
            float* gx = in->requires_grad ? grad_target(in, &ax) : nullptr;
            float* dg = gm->requires_grad ? grad_target(gm, &ag) : nullptr;
            float* db = bt->requires_grad ? grad_target(bt, &ab) : nullptr;
            ck(wm_layernorm_bwd(res->grad.dev(), in->data.dev(), gm->data.dev(), mean->dev(), inv->dev(),
                                (int64_t)rows, (int64_t)n, gx, ax, dg, ag, db, ab),
               "LayerNorm backward");
        };
    }
    return result;
}

std::vector<TensorPtr> LayerNorm::parameters() { return {gamma, beta}; }

// ---- Embedding, LSTM, GRU, MultiHeadAttention: parameters only ------------------------

Embedding::Embedding(size_t num_embeddings, size_t embedding_dim)
    : num_embeddings(num_embeddings), embedding_dim(embedding_dim) {
    weight = Tensor::randn({num_embeddings, embedding_dim}, true);
}

TensorPtr Embedding::forward(const TensorPtr&) { out_of_scope("Embedding::forward"); }
std::vector<TensorPtr> Embedding::parameters() { return {weight}; }

// Recurrent layers: Xavier-style normal weights drawn ih then hh, zero
// biases, the LSTM forget-gate bias set to 1 (core/layer.cpp:570-594, :830-849).
LSTM::LSTM(size_t input_size, size_t hidden_size, bool batch_first)
    : input_size(input_size), hidden_size(hidden_size), batch_first(batch_first) {
    const float std_ih = std::sqrt(2.0f / (input_size + hidden_size));
    const float std_hh = std::sqrt(2.0f / (hidden_size + hidden_size));
    weight_ih = drawn({4 * hidden_size, input_size}, std_ih);
    weight_hh = drawn({4 * hidden_size, hidden_size}, std_hh);
    std::vector<float> bih(4 * hidden_size, 0.0f);
    for (size_t i = hidden_size; i < 2 * hidden_size; ++i) bih[i] = 1.0f;
    bias_ih = Tensor::create(bih, {4 * hidden_size}, true);
    bias_hh = Tensor::zeros({4 * hidden_size}, true);
}

TensorPtr LSTM::forward(const TensorPtr&) { out_of_scope("LSTM::forward"); }
TensorPtr LSTM::forward(const TensorPtr&, const TensorPtr&, const TensorPtr&) { out_of_scope("LSTM::forward"); }
std::vector<TensorPtr> LSTM::parameters() { return {weight_ih, weight_hh, bias_ih, bias_hh}; }

GRU::GRU(size_t input_size, size_t hidden_size, bool batch_first)
    : input_size(input_size), hidden_size(hidden_size), batch_first(batch_first) {
    const float std_ih = std::sqrt(2.0f / (input_size + hidden_size));
    const float std_hh = std::sqrt(2.0f / (hidden_size + hidden_size));
    weight_ih = drawn({3 * hidden_size, input_size}, std_ih);
    weight_hh = drawn({3 * hidden_size, hidden_size}, std_hh);
    bias_ih = Tensor::zeros({3 * hidden_size}, true);
    bias_hh = Tensor::zeros({3 * hidden_size}, true);
}

TensorPtr GRU::forward(const TensorPtr&) { out_of_scope("GRU::forward"); }
TensorPtr GRU::forward(const TensorPtr&, const TensorPtr&) { out_of_scope("GRU::forward"); }
std::vector<TensorPtr> GRU::parameters() { return {weight_ih, weight_hh, bias_ih, bias_hh}; }

// Projections W_q, W_k, W_v, W_o drawn in that order, zero biases
// (core/layer.cpp:1072-1097).
MultiHeadAttention::MultiHeadAttention(size_t embed_dim, size_t num_heads) : embed_dim(embed_dim), num_heads(num_heads) {
    if (num_heads == 0 || embed_dim % num_heads != 0)
        throw std::invalid_argument("MultiHeadAttention: embed_dim must be divisible by num_heads");
    head_dim = embed_dim / num_heads;
    const float sd = std::sqrt(2.0f / (embed_dim + embed_dim));
    W_q = drawn({embed_dim, embed_dim}, sd);
    W_k = drawn({embed_dim, embed_dim}, sd);
    W_v = drawn({embed_dim, embed_dim}, sd);
    W_o = drawn({embed_dim, embed_dim}, sd);
    b_q = Tensor::zeros({embed_dim}, true);
    b_k = Tensor::zeros({embed_dim}, true);
    b_v = Tensor::zeros({embed_dim}, true);
    b_o = Tensor::zeros({embed_dim}, true);
}

TensorPtr MultiHeadAttention::forward(const TensorPtr& input) { return forward(input, input, input, nullptr); }

namespace {
// A gradient buffer to add into: a known-zero buffer is cleared first, since
// wm_mha_bwd only adds.
float* grad_accum_target(const TensorPtr& t) {
    int acc = 0;
    float* g = grad_target(t, &acc);
    if (!acc) ck(wm_fill(g, 0.0f, (int64_t)t->data.size()), "gradient clear");
    return g;
}
}  // namespace

// core/layer.cpp:1103-1437 as wm_mha_fwd / wm_mha_bwd.  The closure exists
// only when an input requires grad (the reference's `track`), and then adds
// into all eight parameter gradients; Q, K, V and the context stay on the
// device for it, attn_weights is the stored attention.
TensorPtr MultiHeadAttention::forward(const TensorPtr& query, const TensorPtr& key, const TensorPtr& value,
                                      const TensorPtr& mask) {
    if (query->shape.size() != 3 || key->shape.size() != 3 || value->shape.size() != 3)
        throw std::invalid_argument("MultiHeadAttention: query, key and value must be 3-D");
    if (query->shape[2] != embed_dim || key->shape[2] != embed_dim || value->shape[2] != embed_dim)
        throw std::invalid_argument("MultiHeadAttention: last dimension must be embed_dim");
    const size_t batch = query->shape[0], seq_q = query->shape[1], seq_k = key->shape[1];
    if (key->shape[0] != batch || value->shape[0] != batch || value->shape[1] != seq_k)
        throw std::invalid_argument("MultiHeadAttention: key / value shapes do not match the query");
    int64_t mask_batches = 0;
    if (mask) {
        const auto& ms = mask->shape;
        if (ms.size() != 4 || (ms[0] != 1 && ms[0] != batch) || ms[1] != 1 || ms[2] != seq_q || ms[3] != seq_k)
            throw std::invalid_argument("MultiHeadAttention: mask must be [batch or 1, 1, seq_q, seq_k]");
        mask_batches = (int64_t)ms[0];
    }
    const bool track = (query->requires_grad || key->requires_grad || value->requires_grad) && GradMode::is_enabled();
    const int64_t B = (int64_t)batch, Sq = (int64_t)seq_q, Sk = (int64_t)seq_k, E = (int64_t)embed_dim,
                  H = (int64_t)num_heads;
    auto Q = std::make_shared<wm::DeviceVector>(batch * seq_q * embed_dim);
    auto K = std::make_shared<wm::DeviceVector>(batch * seq_k * embed_dim);
    auto V = std::make_shared<wm::DeviceVector>(batch * seq_k * embed_dim);
    auto ctx = std::make_shared<wm::DeviceVector>(batch * seq_q * embed_dim);
    auto attn = Tensor::create({batch, num_heads, seq_q, seq_k}, track);
    auto output = Tensor::create({batch, seq_q, embed_dim}, track);
    ck(wm_mha_fwd(query->data.dev(), key->data.dev(), value->data.dev(), mask ? mask->data.dev() : nullptr,
                  mask_batches, W_q->data.dev(), W_k->data.dev(), W_v->data.dev(), W_o->data.dev(), b_q->data.dev(),
                  b_k->data.dev(), b_v->data.dev(), b_o->data.dev(), B, Sq, Sk, E, H, output->data.dev_write(),
                  attn->data.dev_write(), Q->dev_write(), K->dev_write(), V->dev_write(), ctx->dev_write()),
       "MultiHeadAttention");
    attn_weights = attn;
    if (track) {
        TensorPtr q = query, k = key, v = value, Wq = W_q, Wk = W_k, Wv = W_v, Wo = W_o, bq = b_q, bk = b_k, bv = b_v,
                  bo = b_o, at = attn;
        Tensor* out = output.get();
        output->parents = {q, k, v, Wq, Wk, Wv, Wo, bq, bk, bv, bo};
        output->grad_fn = [=]() {
            float* gWq = grad_accum_target(Wq);
            float* gWk = grad_accum_target(Wk);
            float* gWv = grad_accum_target(Wv);
            float* gWo = grad_accum_target(Wo);
            float* gbq = grad_accum_target(bq);
            float* gbk = grad_accum_target(bk);
            float* gbv = grad_accum_target(bv);
            float* gbo = grad_accum_target(bo);
            float* gq = q->requires_grad ? grad_accum_target(q) : nullptr;
            float* gk = k->requires_grad ? (k == q ? gq : grad_accum_target(k)) : nullptr;
            float* gv = nullptr;
            if (v->requires_grad) gv = v == q ? gq : v == k ? gk : grad_accum_target(v);
            ck(wm_mha_bwd(out->grad.dev(), q->data.dev(), k->data.dev(), v->data.dev(), Wq->data.dev(),
                          Wk->data.dev(), Wv->data.dev(), Wo->data.dev(), Q->dev(), K->dev(), V->dev(), at->data.dev(),
                          ctx->dev(), B, Sq, Sk, E, H, gWq, gWk, gWv, gWo, gbq, gbk, gbv, gbo, gq, gk, gv),
               "MultiHeadAttention backward");
        };
    }
    return output;
}

std::vector<TensorPtr> MultiHeadAttention::parameters() { return {W_q, W_k, W_v, W_o, b_q, b_k, b_v, b_o}; }

TensorPtr MultiHeadAttention::causal_mask(size_t seq_len) {
    std::vector<float> m(seq_len * seq_len, 0.0f);
    for (size_t i = 0; i < seq_len; ++i)
        for (size_t j = i + 1; j < seq_len; ++j) m[i * seq_len + j] = -1e9f;
    return Tensor::create(m, {1, 1, seq_len, seq_len}, false);
}

// ---- Sequential (core/layer.cpp:75-130) -------------------------------------------

Sequential::Sequential(std::initializer_list<Module*> modules) : layers(modules) {}

Sequential::~Sequential() {
    for (auto* m : layers) delete m;
}

void Sequential::add(Module* module) { layers.push_back(module); }

TensorPtr Sequential::forward(const TensorPtr& input) {
    TensorPtr x = input;
    for (auto* layer : layers) x = layer->forward(x);
    return x;
}

std::vector<TensorPtr> Sequential::parameters() {
    std::vector<TensorPtr> all;
    for (auto* layer : layers) {
        auto p = layer->parameters();
        all.insert(all.end(), p.begin(), p.end());
    }
    return all;
}

void Sequential::train() {
    for (auto* layer : layers) {
        if (auto* d = dynamic_cast<Dropout*>(layer)) d->train();
        else if (auto* bn = dynamic_cast<BatchNorm2d*>(layer)) bn->train();
    }
}

void Sequential::eval() {
    for (auto* layer : layers) {
        if (auto* d = dynamic_cast<Dropout*>(layer)) d->eval();
        else if (auto* bn = dynamic_cast<BatchNorm2d*>(layer)) bn->eval();
    }
}

// ---- summaries (core/layer.cpp:1471-1826) ---------------------------------------------

std::string Linear::extra_repr() const {
    return "in_features=" + std::to_string(in_features) + ", out_features=" + std::to_string(out_features);
}
std::string Softmax::extra_repr() const { return "dim=" + std::to_string(dim); }
std::string LogSoftmax::extra_repr() const { return "dim=" + std::to_string(dim); }
std::string Dropout::extra_repr() const { return "p=" + std::to_string(p); }
std::string Conv2d::extra_repr() const {
    return std::to_string(in_channels) + ", " + std::to_string(out_channels) +
           ", kernel_size=" + std::to_string(kernel_size) + ", stride=" + std::to_string(stride) +
           ", padding=" + std::to_string(padding);
}
std::string ConvTranspose2d::extra_repr() const {
    return std::to_string(in_channels) + ", " + std::to_string(out_channels) +
           ", kernel_size=" + std::to_string(kernel_size) + ", stride=" + std::to_string(stride) +
           ", padding=" + std::to_string(padding) + ", output_padding=" + std::to_string(output_padding);
}
std::string MaxPool2d::extra_repr() const {
    return "kernel_size=" + std::to_string(kernel_size) + ", stride=" + std::to_string(stride);
}
std::string AvgPool2d::extra_repr() const {
    return "kernel_size=" + std::to_string(kernel_size) + ", stride=" + std::to_string(stride);
}
std::string BatchNorm2d::extra_repr() const {
    return std::to_string(num_features) + ", eps=" + std::to_string(eps) + ", momentum=" + std::to_string(momentum);
}
std::string LayerNorm::extra_repr() const { return shape_str(normalized_shape) + ", eps=" + std::to_string(eps); }
std::string Embedding::extra_repr() const {
    return std::to_string(num_embeddings) + ", " + std::to_string(embedding_dim);
}
std::string LSTM::extra_repr() const {
    return std::to_string(input_size) + ", " + std::to_string(hidden_size) +
           ", batch_first=" + (batch_first ? "true" : "false");
}
std::string GRU::extra_repr() const {
    return std::to_string(input_size) + ", " + std::to_string(hidden_size) +
           ", batch_first=" + (batch_first ? "true" : "false");
}
std::string MultiHeadAttention::extra_repr() const {
    return "embed_dim=" + std::to_string(embed_dim) + ", num_heads=" + std::to_string(num_heads);
}

std::vector<size_t> Linear::compute_output_shape(const std::vector<size_t>& s) const {
    if (s.empty()) return {};
    auto out = s;
    out.back() = out_features;
    return out;
}

std::vector<size_t> Conv2d::compute_output_shape(const std::vector<size_t>& s) const {
    if (s.size() != 4) return s;
    return {s[0], out_channels, (s[2] + 2 * padding - kernel_size) / stride + 1,
            (s[3] + 2 * padding - kernel_size) / stride + 1};
}

std::vector<size_t> ConvTranspose2d::compute_output_shape(const std::vector<size_t>& s) const {
    if (s.size() != 4) return s;
    return {s[0], out_channels, (s[2] - 1) * stride - 2 * padding + kernel_size + output_padding,
            (s[3] - 1) * stride - 2 * padding + kernel_size + output_padding};
}

std::vector<size_t> MaxPool2d::compute_output_shape(const std::vector<size_t>& s) const {
    if (s.size() != 4) return s;
    return {s[0], s[1], (s[2] - kernel_size) / stride + 1, (s[3] - kernel_size) / stride + 1};
}

std::vector<size_t> AvgPool2d::compute_output_shape(const std::vector<size_t>& s) const {
    if (s.size() != 4) return s;
    return {s[0], s[1], (s[2] - kernel_size) / stride + 1, (s[3] - kernel_size) / stride + 1};
}

std::vector<size_t> Flatten::compute_output_shape(const std::vector<size_t>& s) const {
    if (s.size() < 2) return s;
    size_t flat = 1;
    for (size_t i = 1; i < s.size(); ++i) flat *= s[i];
    return {s[0], flat};
}

std::vector<size_t> Embedding::compute_output_shape(const std::vector<size_t>& s) const {
    auto out = s;
    out.push_back(embedding_dim);
    return out;
}

std::vector<size_t> LSTM::compute_output_shape(const std::vector<size_t>& s) const {
    if (s.size() != 3) return s;
    auto out = s;
    out[2] = hidden_size;
    return out;
}

std::vector<size_t> GRU::compute_output_shape(const std::vector<size_t>& s) const {
    if (s.size() != 3) return s;
    auto out = s;
    out[2] = hidden_size;
    return out;
}

void Sequential::summary(const std::vector<size_t>& input_shape) const {
    const char* rule = "==============================================================================\n";
    printf("%s", rule);
    printf("Layer (type)                    Output Shape              Param #\n");
    printf("%s", rule);
    size_t total = 0, trainable = 0;
    std::vector<size_t> shape = input_shape;
    const bool track = !input_shape.empty();
    for (auto* layer : layers) {
        total += layer->num_parameters();
        trainable += layer->num_trainable_parameters();
        std::string out = "-";
        if (track) {
            shape = layer->compute_output_shape(shape);
            out = shape_str(shape);
        }
        std::string label = layer->name();
        const std::string extra = layer->extra_repr();
        if (!extra.empty()) label += "(" + extra + ")";
        if (label.size() > 32) label = label.substr(0, 29) + "...";
        printf("%-32s %-25s %s\n", label.c_str(), out.c_str(), with_commas(layer->num_parameters()).c_str());
    }
    printf("%s", rule);
    printf("Total params: %s\n", with_commas(total).c_str());
    printf("Trainable params: %s\n", with_commas(trainable).c_str());
    printf("Non-trainable params: %s\n", with_commas(total - trainable).c_str());
    printf("%s", rule);
}

std::string format_number(size_t n) { return with_commas(n); }

std::string format_memory(size_t bytes) {
    static const char* units[] = {"B", "KB", "MB", "GB", "TB"};
    int u = 0;
    double size = (double)bytes;
    while (size >= 1024.0 && u < 4) {
        size /= 1024.0;
        ++u;
    }
    char buf[32];
    if (u == 0) snprintf(buf, sizeof(buf), "%zu %s", bytes, units[0]);
    else snprintf(buf, sizeof(buf), "%.2f %s", size, units[u]);
    return buf;
}

ModelSummary get_model_summary(Module* model) {
    ModelSummary s;
    s.total_params = model->num_parameters();
    s.trainable_params = model->num_trainable_parameters();
    s.non_trainable_params = s.total_params - s.trainable_params;
    s.param_memory_bytes = s.total_params * sizeof(float);
    s.param_memory_fp16_bytes = s.total_params * sizeof(uint16_t);
    s.grad_memory_bytes = s.trainable_params * sizeof(float);
    s.total_memory_bytes = s.param_memory_bytes + s.grad_memory_bytes;
    auto* seq = dynamic_cast<Sequential*>(model);
    s.num_layers = seq ? seq->layers.size() : 0;
    return s;
}

void print_model_info(Module* model, const std::string& name) {
    const ModelSummary s = get_model_summary(model);
    const char* rule = "==============================================================================\n";
    const char* thin = "------------------------------------------------------------------------------\n";
    printf("%s%s Summary\n%s", rule, name.c_str(), rule);
    printf("Total parameters:       %s\n", format_number(s.total_params).c_str());
    printf("Trainable parameters:   %s\n", format_number(s.trainable_params).c_str());
    printf("Non-trainable params:   %s\n", format_number(s.non_trainable_params).c_str());
    printf("%s", thin);
    printf("Parameter memory (fp32): %s\n", format_memory(s.param_memory_bytes).c_str());
    printf("Parameter memory (fp16): %s\n", format_memory(s.param_memory_fp16_bytes).c_str());
    printf("Gradient memory:         %s\n", format_memory(s.grad_memory_bytes).c_str());
    printf("Total training memory:   %s\n", format_memory(s.total_memory_bytes).c_str());
    if (s.num_layers > 0) {
        printf("%s", thin);
        printf("Number of layers:        %zu\n", s.num_layers);
    }
    printf("%s", rule);
}
