// ref_shim.cpp -- TEST INFRASTRUCTURE ONLY.
//
// A C entry layer over the reference's own Tensor class (core/tensor.h), so
// that tests and bench.py's cpu_baseline leg can drive the unmodified
// reference CPU path through ctypes.  Built by oracle/Makefile together with
// the reference's core/tensor.cpp (compiled where it lies, with the
// reference's Makefile flags) into oracle/_ref/libwmref.so.
//
// Handles are heap-allocated TensorPtr (std::shared_ptr<Tensor>).
// amp.h uses std::memcpy without including <cstring> itself.
#include <xmmintrin.h>

#include <cstdint>
#include <cstring>
#include <vector>

#include "tensor.h"
#include "amp.h"
#include "optimizer.h"
#include "loss.h"
#include "layer.h"
#include "serialize.h"

#include <memory>

namespace {

// The reference's executables are linked with -ffast-math, whose start-up
// file turns on flush-to-zero and denormals-are-zero for the process.  The
// library is linked without that start-up file (it would change the FP mode
// of every thread that loads it, the oracle's included); instead each entry
// point that runs reference arithmetic switches FTZ/DAZ on for its own
// duration and restores the caller's mode on return.
// The IEEE build (WMREF_IEEE, no fast-math) runs with both modes off.
struct RefFpMode {
    unsigned saved;
#ifdef WMREF_IEEE
    RefFpMode() : saved(_mm_getcsr()) { _mm_setcsr(saved & ~0x8040u); }
#else
    RefFpMode() : saved(_mm_getcsr()) { _mm_setcsr(saved | 0x8040u); }
#endif
    ~RefFpMode() { _mm_setcsr(saved); }
};

TensorPtr& T(void* h) { return *static_cast<TensorPtr*>(h); }
void* box(TensorPtr t) { return new TensorPtr(std::move(t)); }

}  // namespace

extern "C" {

void* wmref_new(const float* data, const int64_t* shape, int nd, int requires_grad) {
    RefFpMode fp_mode_;
    std::vector<size_t> s(shape, shape + nd);
    size_t n = 1;
    for (auto d : s) n *= d;
    std::vector<float> v(data, data + n);
    return box(Tensor::create(v, s, requires_grad != 0));
}

void wmref_free(void* h) { delete static_cast<TensorPtr*>(h); }

int wmref_ndim(void* h) { return (int)T(h)->shape.size(); }

void wmref_shape(void* h, int64_t* out) {
    for (size_t i = 0; i < T(h)->shape.size(); ++i) out[i] = (int64_t)T(h)->shape[i];
}

int64_t wmref_numel(void* h) { return (int64_t)T(h)->data.size(); }

int wmref_requires_grad(void* h) { return T(h)->requires_grad ? 1 : 0; }

void wmref_get_data(void* h, float* out) {
    std::memcpy(out, T(h)->data.data(), T(h)->data.size() * sizeof(float));
}

// Overwrite a tensor's values (its size is unchanged).
void wmref_set_data(void* h, const float* v) {
    std::memcpy(T(h)->data.data(), v, T(h)->data.size() * sizeof(float));
}

// Returns 0 (and writes nothing) when the tensor has no grad buffer.
int wmref_get_grad(void* h, float* out) {
    if (T(h)->grad.empty()) return 0;
    std::memcpy(out, T(h)->grad.data(), T(h)->grad.size() * sizeof(float));
    return 1;
}

// Binary: 0 add, 1 sub, 2 mul, 3 div, 4 pow, 5 max, 6 min (core/tensor.h:73-97).
void* wmref_binary(int op, void* a, void* b) {
    RefFpMode fp_mode_;
    const TensorPtr& x = T(a);
    const TensorPtr& y = T(b);
    switch (op) {
        case 0: return box(x->add(y));
        case 1: return box(x->sub(y));
        case 2: return box(x->mul(y));
        case 3: return box(x->div(y));
        case 4: return box(x->pow(y));
        case 5: return box(x->max(y));
        default: return box(x->min(y));
    }
}

// Tensor::matmul (batched = 0, core/tensor.cpp:783) or Tensor::bmm
// (batched = 1, :827).
void* wmref_matmul(int batched, void* a, void* b) {
    RefFpMode fp_mode_;
    return box(batched ? T(a)->bmm(T(b)) : T(a)->matmul(T(b)));
}

// Unary: 0 relu, 1 sigmoid, 2 tanh_, 3 log_, 4 exp_, 5 pow(p0), 6 sqrt,
// 7 abs, 8 clamp(p0, p1), 9 mul(p0), 10 div(p0), 11 neg.
void* wmref_unary(int op, void* h, float p0, float p1) {
    RefFpMode fp_mode_;
    const TensorPtr& x = T(h);
    switch (op) {
        case 0: return box(x->relu());
        case 1: return box(x->sigmoid());
        case 2: return box(x->tanh_());
        case 3: return box(x->log_());
        case 4: return box(x->exp_());
        case 5: return box(x->pow(p0));
        case 6: return box(x->sqrt());
        case 7: return box(x->abs());
        case 8: return box(x->clamp(p0, p1));
        case 9: return box(x->mul(p0));
        case 10: return box(x->div(p0));
        default: return box(x->neg());
    }
}

// Reductions through the reference API: 0 sum, 1 mean, 2 max, 3 min,
// 4 argmax, 5 argmin (core/tensor.h:92-99).
void* wmref_reduce(int op, void* h, int dim, int keepdim) {
    RefFpMode fp_mode_;
    const TensorPtr& x = T(h);
    bool k = keepdim != 0;
    switch (op) {
        case 0: return box(x->sum(dim, k));
        case 1: return box(x->mean(dim, k));
        case 2: return box(x->max(dim, k));
        case 3: return box(x->min(dim, k));
        case 4: return box(x->argmax(dim, k));
        default: return box(x->argmin(dim, k));
    }
}

void* wmref_softmax(int log, void* h, int dim) {
    RefFpMode fp_mode_;
    return box(log ? T(h)->log_softmax(dim) : T(h)->softmax(dim));
}

void* wmref_reshape(void* h, const int64_t* shape, int nd) {
    RefFpMode fp_mode_;
    std::vector<size_t> s(shape, shape + nd);
    return box(T(h)->reshape(s));
}

// Inject an upstream gradient and run this node's closure only:
// y->grad = g; y->grad_fn().  Returns 0 when the node has no closure.
int wmref_run_grad_fn(void* h, const float* g) {
    RefFpMode fp_mode_;
    TensorPtr& y = T(h);
    if (!y->grad_fn) return 0;
    y->grad.assign(g, g + y->data.size());
    y->grad_fn();
    return 1;
}

// The same in two steps, so a timer can bracket the closure alone.
int wmref_set_grad(void* h, const float* g) {
    RefFpMode fp_mode_;
    TensorPtr& y = T(h);
    y->grad.assign(g, g + y->data.size());
    return y->grad_fn ? 1 : 0;
}

void wmref_call_grad_fn(void* h) {
    RefFpMode fp_mode_;
    T(h)->grad_fn();
}

// Full reverse pass from a scalar root (core/tensor.cpp:763-781).
void wmref_backward(void* h) {
    RefFpMode fp_mode_;
    T(h)->backward();
}

void wmref_zero_grad(void* h) { T(h)->zero_grad(); }

void wmref_set_grad_enabled(int on) { GradMode::set_enabled(on != 0); }

// fp16 storage conversions of core/amp.h:15-72.
void wmref_f32_to_f16(const float* x, uint16_t* out, int64_t n) {
    RefFpMode fp_mode_;
    for (int64_t i = 0; i < n; ++i) out[i] = float_to_half(x[i]);
}

void wmref_f16_to_f32(const uint16_t* x, float* out, int64_t n) {
    RefFpMode fp_mode_;
    for (int64_t i = 0; i < n; ++i) out[i] = half_to_float(x[i]);
}

// ---- parameter updates (core/optimizer.cpp, core/amp.h:125-147) -----------

static std::vector<TensorPtr> param_list(void** params, int np) {
    std::vector<TensorPtr> ps;
    for (int i = 0; i < np; ++i) ps.push_back(T(params[i]));
    return ps;
}

// kind 0: SGD(lr, momentum = a); 1: Adam(lr, beta1 = a, beta2 = b, eps = c);
// 2: AdamW(lr, a, b, c, weight_decay = d); 3: RMSprop(lr, alpha = a, eps = b,
// momentum = c, weight_decay = d).
void* wmref_optim_new(int kind, void** params, int np, float lr, float a, float b, float c, float d) {
    RefFpMode fp_mode_;
    std::vector<TensorPtr> ps = param_list(params, np);
    switch (kind) {
        case 0: return new SGD(ps, lr, a);
        case 1: return new Adam(ps, lr, a, b, c);
        case 2: return new AdamW(ps, lr, a, b, c, d);
        case 3: return new RMSprop(ps, lr, a, b, c, d);
        default: return nullptr;
    }
}

void wmref_optim_step(void* o) {
    RefFpMode fp_mode_;
    static_cast<Optimizer*>(o)->step();
}

void wmref_optim_free(void* o) { delete static_cast<Optimizer*>(o); }

float wmref_grad_norm(void** params, int np) {
    RefFpMode fp_mode_;
    return get_grad_norm(param_list(params, np));
}

void wmref_clip_grad_norm(void** params, int np, float max_norm) {
    RefFpMode fp_mode_;
    std::vector<TensorPtr> ps = param_list(params, np);
    clip_grad_norm_(ps, max_norm);
}

void wmref_clip_grad_value(void** params, int np, float c) {
    RefFpMode fp_mode_;
    std::vector<TensorPtr> ps = param_list(params, np);
    clip_grad_value_(ps, c);
}

// GradScaler(scale).unscale over the params (through an SGD holding them);
// returns 1 when a non-finite gradient stopped it.
int wmref_unscale(void** params, int np, float scale) {
    RefFpMode fp_mode_;
    SGD opt(param_list(params, np), 0.1f);
    GradScaler scaler(scale);
    return scaler.unscale(&opt) ? 0 : 1;
}

// Loss forward through the reference's loss classes (core/loss.h:6-74):
// 0 MSE, 1 L1, 2 SmoothL1(beta = p0), 3 CrossEntropy, 4 NLL, 5 BCE,
// 6 BCEWithLogits, 7 KLDiv(log_target = p0 != 0), 8 Focal(gamma = p0,
// alpha = p1), 9 BinaryFocal(gamma = p0, alpha = p1).  Returns the loss
// tensor; wmref_backward on it runs the closures.
void* wmref_loss(int kind, void* pred, void* target, float p0, float p1) {
    RefFpMode fp_mode_;
    std::unique_ptr<LossFunction> l;
    switch (kind) {
        case 0: l.reset(new MSELoss()); break;
        case 1: l.reset(new L1Loss()); break;
        case 2: l.reset(new SmoothL1Loss(p0)); break;
        case 3: l.reset(new CrossEntropyLoss()); break;
        case 4: l.reset(new NLLLoss()); break;
        case 5: l.reset(new BCELoss()); break;
        case 6: l.reset(new BCEWithLogitsLoss()); break;
        case 7: l.reset(new KLDivLoss(p0 != 0.0f)); break;
        case 8: l.reset(new FocalLoss(p0, p1)); break;
        default: l.reset(new BinaryFocalLoss(p0, p1)); break;
    }
    return box(l->forward(T(pred), T(target)));
}

// Modules of the reference (core/layer.h): 0 LayerNorm(normalized shape,
// eps = p0), 1 BatchNorm2d(num_features = shape[0], eps = p0, momentum =
// p1), 2 MultiHeadAttention(embed_dim = shape[0], num_heads = shape[1]),
// 3 Linear(in_features = shape[0], out_features = shape[1]).
void* wmref_module_new(int kind, const int64_t* shape, int nd, float p0, float p1) {
    RefFpMode fp_mode_;
    std::vector<size_t> s(shape, shape + nd);
    switch (kind) {
        case 0: return new LayerNorm(s, p0);
        case 1: return new BatchNorm2d(s[0], p0, p1);
        case 2: return new MultiHeadAttention(s[0], s[1]);
        default: return new Linear(s[0], s[1]);
    }
}

void wmref_module_free(void* m) { delete static_cast<Module*>(m); }

// BatchNorm2d's training flag.
void wmref_module_train(void* m, int on) {
    if (auto* bn = dynamic_cast<BatchNorm2d*>(static_cast<Module*>(m))) bn->training = on != 0;
}

void* wmref_module_forward(void* m, void* input) {
    RefFpMode fp_mode_;
    return box(static_cast<Module*>(m)->forward(T(input)));
}

// MultiHeadAttention::forward(query, key, value, mask); mask may be NULL.
void* wmref_mha_forward(void* m, void* q, void* k, void* v, void* mask) {
    RefFpMode fp_mode_;
    auto* a = static_cast<MultiHeadAttention*>(static_cast<Module*>(m));
    return box(a->forward(T(q), T(k), T(v), mask ? T(mask) : TensorPtr()));
}

int wmref_module_nparams(void* m) { return (int)static_cast<Module*>(m)->parameters().size(); }

// The i-th parameter tensor (shared with the module).
void* wmref_module_param(void* m, int i) { return box(static_cast<Module*>(m)->parameters()[(size_t)i]); }

// Buffers: BatchNorm2d running_mean (0) / running_var (1); MHA
// attn_weights (0).
void* wmref_module_buffer(void* m, int which) {
    Module* mod = static_cast<Module*>(m);
    if (auto* bn = dynamic_cast<BatchNorm2d*>(mod)) return box(which == 0 ? bn->running_mean : bn->running_var);
    if (auto* a = dynamic_cast<MultiHeadAttention*>(mod)) return box(a->attn_weights);
    return nullptr;
}

// core/serialize.h: the reference's own WMT / WMM / WMO / checkpoint files.
int wmref_save_tensor(void* h, const char* path) { return save_tensor(T(h), std::string(path)) ? 1 : 0; }

void* wmref_load_tensor(const char* path) {
    TensorPtr t = load_tensor(std::string(path));
    return t ? box(t) : nullptr;
}

int wmref_save_model(void* m, const char* path) { return save_model(static_cast<Module*>(m), path) ? 1 : 0; }
int wmref_load_model(void* m, const char* path) { return load_model(static_cast<Module*>(m), path) ? 1 : 0; }
int wmref_save_optimizer(void* o, const char* path) {
    return save_optimizer(static_cast<Optimizer*>(o), path) ? 1 : 0;
}
int wmref_load_optimizer(void* o, const char* path) {
    return load_optimizer(static_cast<Optimizer*>(o), path) ? 1 : 0;
}
int wmref_save_checkpoint(const char* path, void* m, void* o, int epoch, float loss, float acc) {
    return save_checkpoint(path, static_cast<Module*>(m), static_cast<Optimizer*>(o), epoch, loss, acc) ? 1 : 0;
}
int wmref_load_checkpoint(const char* path, void* m, void* o, int* epoch, float* loss, float* acc) {
    Checkpoint info{0, 0.0f, 0.0f};
    const bool ok = load_checkpoint(path, static_cast<Module*>(m), static_cast<Optimizer*>(o), info);
    *epoch = info.epoch;
    *loss = info.loss;
    *acc = info.accuracy;
    return ok ? 1 : 0;
}

// Causal mask, MultiHeadAttention::causal_mask.
void* wmref_causal_mask(int64_t seq_len) { return box(MultiHeadAttention::causal_mask((size_t)seq_len)); }

}  // extern "C"
