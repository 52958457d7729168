// optimizer.cpp -- the drop-in optimizers: step() and the clipping helpers
// run the update kernels of include/wm_optim.h on each parameter's device
// buffers (core/optimizer.cpp:1-177); the schedulers keep the reference's
// host arithmetic (:179-259).
#include "optimizer.h"

#include <memory>
#include <stdexcept>
#include <string>

#include "wm_hip.h"
#include "wm_optim.h"

namespace {

void check(int rc, const char* what) {
    if (rc != WM_OK) throw std::runtime_error(std::string(what) + ": " + wm_last_error());
}

int64_t numel(const TensorPtr& p) { return (int64_t)p->data.size(); }

// One zero-initialised state buffer per parameter.  A fresh DeviceVector of
// zeros is only a flag; the first kernel that writes it materialises it.
std::vector<wm::DeviceVector> zero_state(const std::vector<TensorPtr>& params) {
    std::vector<wm::DeviceVector> s;
    s.reserve(params.size());
    for (const auto& p : params) s.emplace_back(p->data.size(), 0.0f);
    return s;
}

// 1 - beta^t as the reference computes it: std::pow(float, int) is the
// double pow, and the float assignment rounds once (core/optimizer.cpp:48).
float bias_correction(float beta, int t) { return (float)(1.0 - std::pow((double)beta, (double)t)); }

}  // namespace

Optimizer::Optimizer(const std::vector<TensorPtr>& params, float lr) : params(params), lr(lr) {}

void Optimizer::zero_grad() {
    for (auto& p : params) p->zero_grad();
}

namespace {

// The parameter list as the multi-tensor entry points take it: device
// pointers of every parameter's data / grad / state, in parameter order.
struct Lists {
    std::vector<float*> p, s1, s2;
    std::vector<const float*> g;
    std::vector<wm_grad_scale> gs;  // each gradient's deferred scaling (unscale, clip)
    std::vector<int64_t> n;
};

Lists param_lists(std::vector<TensorPtr>& params, std::vector<wm::DeviceVector>* s1,
                  std::vector<wm::DeviceVector>* s2) {
    Lists l;
    l.gs.resize(params.size());
    for (size_t i = 0; i < params.size(); ++i) {
        auto& p = params[i];
        l.n.push_back(numel(p));
        l.p.push_back(p->data.dev_rw());
        l.g.push_back(p->grad.dev_deferred(&l.gs[i]));
        l.s1.push_back(s1 ? (*s1)[i].dev_rw() : nullptr);
        l.s2.push_back(s2 ? (*s2)[i].dev_rw() : nullptr);
    }
    return l;
}

}  // namespace

SGD::SGD(const std::vector<TensorPtr>& params, float lr, float momentum) : Optimizer(params, lr), momentum(momentum) {
    if (momentum > 0.0f) velocity = zero_state(params);
}

// One launch per step over every parameter (core/optimizer.cpp:22-36 per element).
void SGD::step() {
    if (params.empty()) return;
    Lists l = param_lists(params, momentum > 0.0f ? &velocity : nullptr, nullptr);
    check(wm_sgd_step_multi_gs((int)params.size(), l.p.data(), l.g.data(), l.gs.data(),
                               momentum > 0.0f ? l.s1.data() : nullptr, l.n.data(), lr, momentum),
          "SGD::step");
}

Adam::Adam(const std::vector<TensorPtr>& params, float lr, float beta1, float beta2, float eps)
    : Optimizer(params, lr), beta1(beta1), beta2(beta2), eps(eps), t(0), m(zero_state(params)),
      v(zero_state(params)) {}

void Adam::step() {
    ++t;
    if (params.empty()) return;
    Lists l = param_lists(params, &m, &v);
    check(wm_adam_step_multi_gs((int)params.size(), l.p.data(), l.g.data(), l.gs.data(), l.s1.data(), l.s2.data(),
                                l.n.data(), lr, beta1, beta2, eps, bias_correction(beta1, t),
                                bias_correction(beta2, t)),
          "Adam::step");
}

AdamW::AdamW(const std::vector<TensorPtr>& params, float lr, float beta1, float beta2, float eps, float weight_decay)
    : Optimizer(params, lr), beta1(beta1), beta2(beta2), eps(eps), weight_decay(weight_decay), t(0),
      m(zero_state(params)), v(zero_state(params)) {}

void AdamW::step() {
    ++t;
    if (params.empty()) return;
    Lists l = param_lists(params, &m, &v);
    check(wm_adamw_step_multi_gs((int)params.size(), l.p.data(), l.g.data(), l.gs.data(), l.s1.data(), l.s2.data(),
                                 l.n.data(), lr, beta1, beta2, eps, bias_correction(beta1, t),
                                 bias_correction(beta2, t), weight_decay),
          "AdamW::step");
}

RMSprop::RMSprop(const std::vector<TensorPtr>& params, float lr, float alpha, float eps, float momentum,
                 float weight_decay)
    : Optimizer(params, lr), alpha(alpha), eps(eps), momentum(momentum), weight_decay(weight_decay),
      v(zero_state(params)) {
    if (momentum > 0.0f) buffer = zero_state(params);
}

void RMSprop::step() {
    if (params.empty()) return;
    Lists l = param_lists(params, &v, momentum > 0.0f ? &buffer : nullptr);
    check(wm_rmsprop_step_multi_gs((int)params.size(), l.p.data(), l.g.data(), l.gs.data(), l.s1.data(),
                                   momentum > 0.0f ? l.s2.data() : nullptr, l.n.data(), lr, alpha, eps, momentum,
                                   weight_decay),
          "RMSprop::step");
}

// ---- clipping ---------------------------------------------------------------

namespace {

// Every non-empty gradient of the list, for the multi-tensor calls (a
// parameter whose grad is empty contributes nothing, as in the reference's
// loops over grad.size()).
struct GradList {
    std::vector<float*> g;
    std::vector<int64_t> n;
};

GradList grad_list(const std::vector<TensorPtr>& params, bool write) {
    GradList l;
    for (const auto& p : params) {
        if (p->grad.empty()) continue;
        l.g.push_back(write ? p->grad.dev_rw() : const_cast<float*>(p->grad.dev()));
        l.n.push_back((int64_t)p->grad.size());
    }
    return l;
}

// get_grad_norm's sum of squares (core/optimizer.cpp:145-153) into a
// one-element device buffer, over the gradients' current values (their
// deferred scalings applied as they are read).
std::shared_ptr<wm::DeviceVector> grad_sumsq(const std::vector<TensorPtr>& params) {
    auto total = std::make_shared<wm::DeviceVector>(1, 0.0f);
    std::vector<const float*> g;
    std::vector<wm_grad_scale> gs;
    std::vector<int64_t> n;
    for (const auto& p : params) {
        if (p->grad.empty()) continue;
        gs.emplace_back();
        g.push_back(p->grad.dev_deferred(&gs.back()));
        n.push_back((int64_t)p->grad.size());
    }
    if (g.empty()) return total;  // known zero
    check(wm_grad_sumsq_multi_gs((int)g.size(), g.data(), gs.data(), n.data(), 1.0f, total->dev_write()),
          "get_grad_norm");
    return total;
}

}  // namespace

float get_grad_norm(const std::vector<TensorPtr>& params) {
    const auto total = grad_sumsq(params);
    return std::sqrt((*total)[0]);
}

// The norm is one read of every gradient; the multiplication by the clip
// coefficient is deferred (DeviceVector::defer_clip): the coefficient is
// computed on the device from the device-side norm when the scaling is
// applied -- by the optimizer step that reads the gradients next, or one
// pass before any other use -- so clipping never waits for the host and
// costs no second pass over the gradients before a step.
void clip_grad_norm_(std::vector<TensorPtr>& params, float max_norm) {
    const auto total = grad_sumsq(params);
    for (auto& p : params)
        if (!p->grad.empty()) p->grad.defer_clip(total, max_norm);
}

void clip_grad_value_(std::vector<TensorPtr>& params, float clip_value) {
    GradList l = grad_list(params, true);
    if (!l.g.empty())
        check(wm_clip_grad_value_multi((int)l.g.size(), l.g.data(), l.n.data(), clip_value), "clip_grad_value_");
}

// ---- schedulers (host arithmetic, core/optimizer.cpp:179-259) ----------------

LRScheduler::LRScheduler(Optimizer* optimizer) : optimizer(optimizer), base_lr(optimizer->lr), last_epoch(-1) {}

void LRScheduler::step() {
    ++last_epoch;
    optimizer->lr = get_lr();
}

StepLR::StepLR(Optimizer* optimizer, int step_size, float gamma)
    : LRScheduler(optimizer), step_size(step_size), gamma(gamma) {}

float StepLR::get_lr() {
    return last_epoch == -1 ? base_lr : base_lr * std::pow(gamma, last_epoch / step_size);
}

ExponentialLR::ExponentialLR(Optimizer* optimizer, float gamma) : LRScheduler(optimizer), gamma(gamma) {}

float ExponentialLR::get_lr() { return last_epoch == -1 ? base_lr : base_lr * std::pow(gamma, last_epoch); }

CosineAnnealingLR::CosineAnnealingLR(Optimizer* optimizer, int T_max, float eta_min)
    : LRScheduler(optimizer), T_max(T_max), eta_min(eta_min) {}

float CosineAnnealingLR::get_lr() {
    if (last_epoch == -1) return base_lr;
    return eta_min + (base_lr - eta_min) * (1.0f + std::cos(M_PI * last_epoch / T_max)) / 2.0f;
}

CosineAnnealingWarmRestarts::CosineAnnealingWarmRestarts(Optimizer* optimizer, int T_0, int T_mult, float eta_min)
    : LRScheduler(optimizer), T_0(T_0), T_mult(T_mult), eta_min(eta_min), T_cur(0), T_i(T_0) {}

float CosineAnnealingWarmRestarts::get_lr() {
    return eta_min + (base_lr - eta_min) * (1.0f + std::cos(M_PI * T_cur / T_i)) / 2.0f;
}

void CosineAnnealingWarmRestarts::step() {
    ++last_epoch;
    if (++T_cur >= T_i) {
        T_cur = 0;
        T_i *= T_mult;
    }
    optimizer->lr = get_lr();
}

ReduceLROnPlateau::ReduceLROnPlateau(Optimizer* optimizer, float factor, int patience, float min_lr, bool mode_min)
    : optimizer(optimizer), factor(factor), patience(patience), min_lr(min_lr), num_bad_epochs(0),
      best(mode_min ? 1e10f : -1e10f), mode_min(mode_min) {}

void ReduceLROnPlateau::step(float metric) {
    if (mode_min ? metric < best : metric > best) {
        best = metric;
        num_bad_epochs = 0;
    } else {
        ++num_bad_epochs;
    }
    if (num_bad_epochs > patience) {
        const float reduced = optimizer->lr * factor;
        if (reduced >= min_lr) optimizer->lr = reduced;
        num_bad_epochs = 0;
    }
}
