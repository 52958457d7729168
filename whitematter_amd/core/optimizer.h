// optimizer.h -- drop-in for whitematter's core/optimizer.h with the
// parameter updates on the GPU.
//
// Same classes, members, signatures, defaults and include guard as the
// reference header (core/optimizer.h:1-419), so code written against it
// compiles unchanged.  What differs is where things live:
//   - the optimizer state (SGD::velocity, Adam/AdamW::m and v,
//     RMSprop::v and buffer) is one DeviceVector per parameter instead of a
//     std::vector<float>: it stays in HBM across steps, and host code that
//     reads or writes it (checkpointing: core/serialize.cpp:205-230) goes
//     through DeviceVector's coherent vector API;
//   - step(), clip_grad_norm_, clip_grad_value_ and get_grad_norm run the
//     kernels of include/wm_optim.h on the parameters' device buffers.
// The learning-rate schedulers, ReduceLROnPlateau, EarlyStopping,
// ModelCheckpoint and GradientAccumulator are host bookkeeping; they keep the
// reference's behaviour.
#ifndef OPTIMIZER_H
#define OPTIMIZER_H

#include "tensor.h"

#include <cmath>
#include <limits>
#include <string>
#include <vector>

class Module;
bool save_model(Module* module, const std::string& path);
bool load_model(Module* module, const std::string& path);

class Optimizer {
public:
    std::vector<TensorPtr> params;
    float lr;

    Optimizer(const std::vector<TensorPtr>& params, float lr);
    virtual ~Optimizer() = default;

    virtual void step() = 0;
    void zero_grad();
};

class SGD : public Optimizer {
public:
    float momentum;
    std::vector<wm::DeviceVector> velocity;  // one per parameter, only when momentum > 0

    SGD(const std::vector<TensorPtr>& params, float lr, float momentum = 0.0f);
    void step() override;
};

class Adam : public Optimizer {
public:
    float beta1, beta2, eps;
    int t;
    std::vector<wm::DeviceVector> m;
    std::vector<wm::DeviceVector> v;

    Adam(const std::vector<TensorPtr>& params, float lr = 0.001f, float beta1 = 0.9f, float beta2 = 0.999f,
         float eps = 1e-8f);
    void step() override;
};

class AdamW : public Optimizer {
public:
    float beta1, beta2, eps, weight_decay;
    int t;
    std::vector<wm::DeviceVector> m;
    std::vector<wm::DeviceVector> v;

    AdamW(const std::vector<TensorPtr>& params, float lr = 0.001f, float beta1 = 0.9f, float beta2 = 0.999f,
          float eps = 1e-8f, float weight_decay = 0.01f);
    void step() override;
};

class RMSprop : public Optimizer {
public:
    float alpha, eps, momentum, weight_decay;
    std::vector<wm::DeviceVector> v;
    std::vector<wm::DeviceVector> buffer;  // only when momentum > 0

    RMSprop(const std::vector<TensorPtr>& params, float lr = 0.01f, float alpha = 0.99f, float eps = 1e-8f,
            float momentum = 0.0f, float weight_decay = 0.0f);
    void step() override;
};

// Gradient clipping (core/optimizer.cpp:141-177)
void clip_grad_norm_(std::vector<TensorPtr>& params, float max_norm);
void clip_grad_value_(std::vector<TensorPtr>& params, float clip_value);
float get_grad_norm(const std::vector<TensorPtr>& params);

// Gradient accumulation over several mini-batches (core/optimizer.h:84-158):
// the loss is scaled by 1/accumulation_steps and the caller steps the
// optimizer once every accumulation_steps backward passes.
class GradientAccumulator {
public:
    explicit GradientAccumulator(int accumulation_steps)
        : accumulation_steps_(accumulation_steps < 1 ? 1 : accumulation_steps),
          current_step_(0),
          scale_factor_(accumulation_steps < 1 ? 1.0f : 1.0f / accumulation_steps) {}

    TensorPtr scale(const TensorPtr& loss) const {
        return accumulation_steps_ == 1 ? loss : loss->mul(scale_factor_);
    }
    void backward(const TensorPtr& loss) {
        scale(loss)->backward();
        ++current_step_;
    }
    bool should_step() const { return current_step_ >= accumulation_steps_; }
    void increment() { ++current_step_; }
    void reset() { current_step_ = 0; }
    int current_step() const { return current_step_; }
    int get_accumulation_steps() const { return accumulation_steps_; }
    float get_scale_factor() const { return scale_factor_; }
    bool is_last_step() const { return current_step_ == accumulation_steps_ - 1; }

private:
    int accumulation_steps_;
    int current_step_;
    float scale_factor_;
};

// Learning-rate schedulers (core/optimizer.h:160-230, core/optimizer.cpp:183-259)
class LRScheduler {
public:
    Optimizer* optimizer;
    float base_lr;
    int last_epoch;

    LRScheduler(Optimizer* optimizer);
    virtual ~LRScheduler() = default;

    virtual void step();
    virtual float get_lr() = 0;
    float get_last_lr() const { return optimizer->lr; }
};

class StepLR : public LRScheduler {
public:
    int step_size;
    float gamma;

    StepLR(Optimizer* optimizer, int step_size, float gamma = 0.1f);
    float get_lr() override;
};

class ExponentialLR : public LRScheduler {
public:
    float gamma;

    ExponentialLR(Optimizer* optimizer, float gamma);
    float get_lr() override;
};

class CosineAnnealingLR : public LRScheduler {
public:
    int T_max;
    float eta_min;

    CosineAnnealingLR(Optimizer* optimizer, int T_max, float eta_min = 0.0f);
    float get_lr() override;
};

class CosineAnnealingWarmRestarts : public LRScheduler {
public:
    int T_0;
    int T_mult;
    float eta_min;
    int T_cur;
    int T_i;

    CosineAnnealingWarmRestarts(Optimizer* optimizer, int T_0, int T_mult = 1, float eta_min = 0.0f);
    float get_lr() override;
    void step() override;
};

class ReduceLROnPlateau {
public:
    Optimizer* optimizer;
    float factor;
    int patience;
    float min_lr;
    int num_bad_epochs;
    float best;
    bool mode_min;

    ReduceLROnPlateau(Optimizer* optimizer, float factor = 0.1f, int patience = 10, float min_lr = 0.0f,
                      bool mode_min = true);
    void step(float metric);
};

// Early stopping on a monitored metric (core/optimizer.h:254-356).  The first
// metric seeds the best value unless a baseline is given; patience
// consecutive non-improving steps stop training.  In mode_min an improvement
// is metric < best - min_delta.  For mode max the reference stores -min_delta
// and then adds it (core/optimizer.h:270-273, :291-293), so an improvement there
// is metric > best - min_delta; that behaviour is kept.
class EarlyStopping {
public:
    EarlyStopping(int patience = 10, float min_delta = 0.0f, bool mode_min = true,
                  float baseline = std::numeric_limits<float>::quiet_NaN())
        : patience_(patience), min_delta_(mode_min ? min_delta : -min_delta), mode_min_(mode_min), counter_(0),
          best_(baseline), best_epoch_(-1), stopped_epoch_(-1), should_stop_(false) {}

    bool step(float metric) {
        if (should_stop_) return true;
        if (std::isnan(best_)) {
            best_ = metric;
            best_epoch_ = 0;
            return false;
        }
        const bool improved = mode_min_ ? metric < best_ - min_delta_ : metric > best_ + min_delta_;
        if (improved) {
            best_epoch_ += counter_ + 1;
            best_ = metric;
            counter_ = 0;
        } else if (++counter_ >= patience_) {
            should_stop_ = true;
            stopped_epoch_ = best_epoch_ + counter_;
        }
        return should_stop_;
    }

    void reset() {
        counter_ = 0;
        best_ = std::numeric_limits<float>::quiet_NaN();
        best_epoch_ = -1;
        stopped_epoch_ = -1;
        should_stop_ = false;
    }

    bool should_stop() const { return should_stop_; }
    float best_metric() const { return best_; }
    int best_epoch() const { return best_epoch_; }
    int stopped_epoch() const { return stopped_epoch_; }
    int patience() const { return patience_; }
    int epochs_without_improvement() const { return counter_; }
    void set_patience(int p) { patience_ = p; }

private:
    int patience_;
    float min_delta_;
    bool mode_min_;
    int counter_;
    float best_;
    int best_epoch_;
    int stopped_epoch_;
    bool should_stop_;
};

// Saves the model whenever the metric improves by more than min_delta
// (core/optimizer.h:358-417).
class ModelCheckpoint {
public:
    ModelCheckpoint(const std::string& filepath, bool mode_min = true, float min_delta = 0.0f)
        : filepath_(filepath), mode_min_(mode_min), min_delta_(min_delta), best_(worst(mode_min)), saved_(false) {}

    bool step(float metric, Module* model) {
        const bool improved = mode_min_ ? metric < best_ - min_delta_ : metric > best_ + min_delta_;
        if (!improved) return false;
        best_ = metric;
        save_model(model, filepath_);
        saved_ = true;
        return true;
    }

    bool restore(Module* model) {
        if (!saved_) return false;
        load_model(model, filepath_);
        return true;
    }

    float best_metric() const { return best_; }
    bool has_saved() const { return saved_; }
    const std::string& filepath() const { return filepath_; }
    void reset() {
        best_ = worst(mode_min_);
        saved_ = false;
    }

private:
    static float worst(bool mode_min) {
        return mode_min ? std::numeric_limits<float>::infinity() : -std::numeric_limits<float>::infinity();
    }

    std::string filepath_;
    bool mode_min_;
    float min_delta_;
    float best_;
    bool saved_;
};

#endif  // OPTIMIZER_H
