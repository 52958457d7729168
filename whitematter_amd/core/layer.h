// layer.h -- drop-in for whitematter's core/layer.h on MI355X.
//
// Same classes, members, constructors, defaults, virtual interface, summary
// utilities and include guard as the reference header (core/layer.h:1-375),
// so code written against it compiles unchanged.  What runs where:
//   - LayerNorm and BatchNorm2d run the kernels of include/wm_layers.h
//     (forward, running statistics, and a backward closure on the device);
//   - MultiHeadAttention runs wm_mha_fwd / wm_mha_bwd (projections and
//     per-head products on the matrix cores, the attention softmax kernels);
//   - Linear, ReLU, Sigmoid, Tanh, Softmax, LogSoftmax, Flatten are the same
//     Tensor ops as in the reference (Linear: matmul then add), so they run
//     on the device through tensor.h;
//   - Dropout multiplies by a device-drawn mask (wm_dropout_mask);
//   - Conv2d, ConvTranspose2d, MaxPool2d and AvgPool2d call the same Tensor
//     ops as the reference (conv2d, pools), which this build's Tensor does
//     not provide (they throw); Embedding, LSTM and GRU need gather / gate
//     kernels this build does not have and throw from forward().  Their
//     constructors, parameters and summaries behave as the reference's,
//     including the seeded initialisation (one std::mt19937(123) shared by
//     all constructors).
#ifndef LAYER_H
#define LAYER_H

#include <initializer_list>
#include <string>
#include <vector>

#include "tensor.h"

class Module {
public:
    virtual ~Module() = default;
    virtual TensorPtr forward(const TensorPtr& input) = 0;
    virtual std::vector<TensorPtr> parameters() { return {}; }

    virtual size_t num_parameters() const;
    virtual size_t num_trainable_parameters() const;

    virtual std::string name() const { return "Module"; }
    virtual std::string extra_repr() const { return ""; }

    // Output shape for summaries (default: unchanged).
    virtual std::vector<size_t> compute_output_shape(const std::vector<size_t>& input_shape) const {
        return input_shape;
    }

    TensorPtr operator()(const TensorPtr& input) { return forward(input); }
};

class Linear : public Module {
public:
    TensorPtr weight;
    TensorPtr bias;
    size_t in_features, out_features;

    Linear(size_t in_features, size_t out_features);

    TensorPtr forward(const TensorPtr& input) override;
    std::vector<TensorPtr> parameters() override;
    std::string name() const override { return "Linear"; }
    std::string extra_repr() const override;
    std::vector<size_t> compute_output_shape(const std::vector<size_t>& input_shape) const override;
};

class ReLU : public Module {
public:
    TensorPtr forward(const TensorPtr& input) override;
    std::string name() const override { return "ReLU"; }
};

class Sigmoid : public Module {
public:
    TensorPtr forward(const TensorPtr& input) override;
    std::string name() const override { return "Sigmoid"; }
};

class Tanh : public Module {
public:
    TensorPtr forward(const TensorPtr& input) override;
    std::string name() const override { return "Tanh"; }
};

class Softmax : public Module {
public:
    int dim;
    Softmax(int dim = -1);
    TensorPtr forward(const TensorPtr& input) override;
    std::string name() const override { return "Softmax"; }
    std::string extra_repr() const override;
};

class LogSoftmax : public Module {
public:
    int dim;
    LogSoftmax(int dim = -1);
    TensorPtr forward(const TensorPtr& input) override;
    std::string name() const override { return "LogSoftmax"; }
    std::string extra_repr() const override;
};

class Dropout : public Module {
public:
    float p;
    bool training;

    Dropout(float p = 0.5f);
    TensorPtr forward(const TensorPtr& input) override;
    void train() { training = true; }
    void eval() { training = false; }
    std::string name() const override { return "Dropout"; }
    std::string extra_repr() const override;
};

class Conv2d : public Module {
public:
    TensorPtr weight;
    TensorPtr bias;
    size_t in_channels, out_channels;
    size_t kernel_size;
    size_t stride;
    size_t padding;

    Conv2d(size_t in_channels, size_t out_channels, size_t kernel_size, size_t stride = 1, size_t padding = 0);

    TensorPtr forward(const TensorPtr& input) override;
    std::vector<TensorPtr> parameters() override;
    std::string name() const override { return "Conv2d"; }
    std::string extra_repr() const override;
    std::vector<size_t> compute_output_shape(const std::vector<size_t>& input_shape) const override;
};

class ConvTranspose2d : public Module {
public:
    TensorPtr weight;
    TensorPtr bias;
    size_t in_channels, out_channels;
    size_t kernel_size;
    size_t stride;
    size_t padding;
    size_t output_padding;

    ConvTranspose2d(size_t in_channels, size_t out_channels, size_t kernel_size, size_t stride = 1,
                    size_t padding = 0, size_t output_padding = 0);

    TensorPtr forward(const TensorPtr& input) override;
    std::vector<TensorPtr> parameters() override;
    std::string name() const override { return "ConvTranspose2d"; }
    std::string extra_repr() const override;
    std::vector<size_t> compute_output_shape(const std::vector<size_t>& input_shape) const override;
};

class MaxPool2d : public Module {
public:
    size_t kernel_size;
    size_t stride;

    MaxPool2d(size_t kernel_size, size_t stride = 0);
    TensorPtr forward(const TensorPtr& input) override;
    std::string name() const override { return "MaxPool2d"; }
    std::string extra_repr() const override;
    std::vector<size_t> compute_output_shape(const std::vector<size_t>& input_shape) const override;
};

class AvgPool2d : public Module {
public:
    size_t kernel_size;
    size_t stride;

    AvgPool2d(size_t kernel_size, size_t stride = 0);
    TensorPtr forward(const TensorPtr& input) override;
    std::string name() const override { return "AvgPool2d"; }
    std::string extra_repr() const override;
    std::vector<size_t> compute_output_shape(const std::vector<size_t>& input_shape) const override;
};

class BatchNorm2d : public Module {
public:
    size_t num_features;
    float eps;
    float momentum;
    bool training;

    TensorPtr gamma;  // scale
    TensorPtr beta;   // shift
    TensorPtr running_mean;
    TensorPtr running_var;

    BatchNorm2d(size_t num_features, float eps = 1e-5f, float momentum = 0.1f);

    TensorPtr forward(const TensorPtr& input) override;
    std::vector<TensorPtr> parameters() override;
    void train() { training = true; }
    void eval() { training = false; }
    std::string name() const override { return "BatchNorm2d"; }
    std::string extra_repr() const override;
};

class LayerNorm : public Module {
public:
    std::vector<size_t> normalized_shape;
    float eps;

    TensorPtr gamma;  // scale
    TensorPtr beta;   // shift

    LayerNorm(std::vector<size_t> normalized_shape, float eps = 1e-5f);
    LayerNorm(size_t normalized_shape, float eps = 1e-5f);

    TensorPtr forward(const TensorPtr& input) override;
    std::vector<TensorPtr> parameters() override;
    std::string name() const override { return "LayerNorm"; }
    std::string extra_repr() const override;
};

class Flatten : public Module {
public:
    TensorPtr forward(const TensorPtr& input) override;
    std::string name() const override { return "Flatten"; }
    std::vector<size_t> compute_output_shape(const std::vector<size_t>& input_shape) const override;
};

class Embedding : public Module {
public:
    TensorPtr weight;
    size_t num_embeddings;
    size_t embedding_dim;

    Embedding(size_t num_embeddings, size_t embedding_dim);

    TensorPtr forward(const TensorPtr& indices) override;
    std::vector<TensorPtr> parameters() override;
    std::string name() const override { return "Embedding"; }
    std::string extra_repr() const override;
    std::vector<size_t> compute_output_shape(const std::vector<size_t>& input_shape) const override;
};

class LSTM : public Module {
public:
    size_t input_size;
    size_t hidden_size;
    bool batch_first;

    // [4*hidden, input] and [4*hidden, hidden]; gates i, f, g, o
    TensorPtr weight_ih;
    TensorPtr weight_hh;
    TensorPtr bias_ih;
    TensorPtr bias_hh;

    TensorPtr h_n;
    TensorPtr c_n;

    LSTM(size_t input_size, size_t hidden_size, bool batch_first = true);

    TensorPtr forward(const TensorPtr& input) override;
    TensorPtr forward(const TensorPtr& input, const TensorPtr& h0, const TensorPtr& c0);

    std::vector<TensorPtr> parameters() override;
    std::string name() const override { return "LSTM"; }
    std::string extra_repr() const override;
    std::vector<size_t> compute_output_shape(const std::vector<size_t>& input_shape) const override;
};

class GRU : public Module {
public:
    size_t input_size;
    size_t hidden_size;
    bool batch_first;

    // [3*hidden, input] and [3*hidden, hidden]; gates r, z, n
    TensorPtr weight_ih;
    TensorPtr weight_hh;
    TensorPtr bias_ih;
    TensorPtr bias_hh;

    TensorPtr h_n;

    GRU(size_t input_size, size_t hidden_size, bool batch_first = true);

    TensorPtr forward(const TensorPtr& input) override;
    TensorPtr forward(const TensorPtr& input, const TensorPtr& h0);

    std::vector<TensorPtr> parameters() override;
    std::string name() const override { return "GRU"; }
    std::string extra_repr() const override;
    std::vector<size_t> compute_output_shape(const std::vector<size_t>& input_shape) const override;
};

class MultiHeadAttention : public Module {
public:
    size_t embed_dim;
    size_t num_heads;
    size_t head_dim;

    TensorPtr W_q, W_k, W_v, W_o;
    TensorPtr b_q, b_k, b_v, b_o;

    TensorPtr attn_weights;

    MultiHeadAttention(size_t embed_dim, size_t num_heads);

    TensorPtr forward(const TensorPtr& input) override;
    TensorPtr forward(const TensorPtr& query, const TensorPtr& key, const TensorPtr& value,
                      const TensorPtr& mask = nullptr);

    std::vector<TensorPtr> parameters() override;
    std::string name() const override { return "MultiHeadAttention"; }
    std::string extra_repr() const override;

    // [1, 1, seq_len, seq_len]: 0 on and below the diagonal, -1e9 above.
    static TensorPtr causal_mask(size_t seq_len);
};

class Sequential : public Module {
public:
    std::vector<Module*> layers;

    Sequential() = default;
    Sequential(std::initializer_list<Module*> modules);
    ~Sequential();

    void add(Module* module);
    TensorPtr forward(const TensorPtr& input) override;
    std::vector<TensorPtr> parameters() override;
    std::string name() const override { return "Sequential"; }

    void train();
    void eval();

    void summary(const std::vector<size_t>& input_shape = {}) const;
};

// ---- model summary utilities (core/layer.h:338-373) ------------------------

struct ModelSummary {
    size_t total_params;
    size_t trainable_params;
    size_t non_trainable_params;
    size_t param_memory_bytes;
    size_t param_memory_fp16_bytes;
    size_t grad_memory_bytes;
    size_t total_memory_bytes;
    size_t num_layers;
};

ModelSummary get_model_summary(Module* model);

inline size_t count_parameters(Module* model) { return model->num_parameters(); }
inline size_t count_trainable_parameters(Module* model) { return model->num_trainable_parameters(); }

std::string format_memory(size_t bytes);
std::string format_number(size_t n);
void print_model_info(Module* model, const std::string& name = "Model");

#endif  // LAYER_H
