// loss.cpp -- the drop-in losses: each forward and its backward closure run
// the device entry points of include/wm_loss.h on the prediction's and
// target's device buffers (reference core/loss.cpp:1-418).
//
// Graph structure: every loss tensor has requires_grad = the prediction's
// (the reference does not consult GradMode here) and, when set, the
// prediction as its only parent.  The reference's CrossEntropyLoss routes its
// gradient through an intermediate log_softmax tensor (loss.cpp:74, :86); the
// fused head computes the same gradient directly into the prediction, so that
// intermediate is never materialised.  MSELoss and L1Loss are compositions of
// Tensor ops in the reference and stay so.
#include "loss.h"

#include <memory>
#include <stdexcept>
#include <string>

#include "wm_hip.h"
#include "wm_loss.h"

namespace {

void ck(int rc, const char* what) {
    if (rc != WM_OK) throw std::runtime_error(std::string("whitematter_amd ") + what + ": " + wm_last_error());
}

// A gradient buffer sized like the tensor's data (the reference allocates it
// at creation when requires_grad is set).
float* grad_target(const TensorPtr& t, int* accumulate) {
    if (t->grad.size() != t->data.size()) t->grad = wm::DeviceVector(t->data.size());
    return t->grad.dev_accum(accumulate);
}

// The shapes a classification head accepts (loss.cpp:68-69, :100-101,
// :264-265): a [batch, classes] prediction and a [batch] or [batch, 1]
// target of class indices.  The reference asserts the first two and reads
// batch entries of the target; a shorter target is rejected here.
void check_head(const TensorPtr& pred, const TensorPtr& target, const char* what) {
    if (pred->shape.size() != 2)
        throw std::invalid_argument(std::string(what) + ": prediction must be [batch, classes]");
    if (!(target->shape.size() == 1 || (target->shape.size() == 2 && target->shape[1] == 1)))
        throw std::invalid_argument(std::string(what) + ": target must be [batch] or [batch, 1]");
    if (target->data.size() < pred->shape[0])
        throw std::invalid_argument(std::string(what) + ": target has fewer entries than the batch");
}

void check_same_size(const TensorPtr& pred, const TensorPtr& target, const char* what) {
    if (pred->data.size() != target->data.size())
        throw std::invalid_argument(std::string(what) + ": prediction and target sizes differ");
}

// The element-wise losses: one forward launch, one backward launch.
TensorPtr pointwise(int kind, const TensorPtr& pred, const TensorPtr& target, float p0, float p1, float denom,
                    const char* what) {
    check_same_size(pred, target, what);
    const int64_t n = (int64_t)pred->data.size();
    auto result = Tensor::create({1}, pred->requires_grad);
    ck(wm_pointwise_loss_fwd(kind, pred->data.dev(), target->data.dev(), n, p0, p1, denom,
                             result->data.dev_write()),
       what);
    if (result->requires_grad) {
        Tensor* res = result.get();
        result->parents = {pred};
        result->grad_fn = [pred, target, res, kind, n, p0, p1, denom, what]() {
            int acc = 0;
            float* gx = grad_target(pred, &acc);
            ck(wm_pointwise_loss_bwd(kind, pred->data.dev(), target->data.dev(), n, p0, p1, denom, res->grad.dev(),
                                     gx, acc),
               what);
        };
    }
    return result;
}

}  // namespace

// ---- compositions of Tensor ops (loss.cpp:4-19) ------------------------------

TensorPtr MSELoss::forward(const TensorPtr& prediction, const TensorPtr& target) {
    check_same_size(prediction, target, "MSELoss");
    auto diff = prediction->sub(target);
    return diff->mul(diff)->mean();
}

TensorPtr L1Loss::forward(const TensorPtr& prediction, const TensorPtr& target) {
    check_same_size(prediction, target, "L1Loss");
    return prediction->sub(target)->abs()->mean();
}

// ---- element-wise losses -----------------------------------------------------

TensorPtr SmoothL1Loss::forward(const TensorPtr& prediction, const TensorPtr& target) {
    return pointwise(WM_L_SMOOTH_L1, prediction, target, beta, 0.0f, (float)prediction->data.size(), "SmoothL1Loss");
}

TensorPtr BCELoss::forward(const TensorPtr& prediction, const TensorPtr& target) {
    return pointwise(WM_L_BCE, prediction, target, 0.0f, 0.0f, (float)prediction->data.size(), "BCELoss");
}

TensorPtr BCEWithLogitsLoss::forward(const TensorPtr& prediction, const TensorPtr& target) {
    return pointwise(WM_L_BCE_LOGITS, prediction, target, 0.0f, 0.0f, (float)prediction->data.size(),
                     "BCEWithLogitsLoss");
}

// Divides by the batch size, prediction->shape[0] (loss.cpp:209-210, :236).
TensorPtr KLDivLoss::forward(const TensorPtr& prediction, const TensorPtr& target) {
    if (prediction->shape.empty()) throw std::invalid_argument("KLDivLoss: prediction needs a batch dimension");
    return pointwise(log_target ? WM_L_KLDIV_LOG : WM_L_KLDIV, prediction, target, 0.0f, 0.0f,
                     (float)prediction->shape[0], "KLDivLoss");
}

TensorPtr BinaryFocalLoss::forward(const TensorPtr& prediction, const TensorPtr& target) {
    return pointwise(WM_L_BINARY_FOCAL, prediction, target, gamma, alpha, (float)prediction->data.size(),
                     "BinaryFocalLoss");
}

// ---- classification heads -----------------------------------------------------

// loss.cpp:67-97: log_softmax, label gather and batch mean in one row pass;
// the backward is the label scatter followed by log_softmax's closure, fused.
TensorPtr CrossEntropyLoss::forward(const TensorPtr& prediction, const TensorPtr& target) {
    check_head(prediction, target, "CrossEntropyLoss");
    const int64_t rows = (int64_t)prediction->shape[0], cols = (int64_t)prediction->shape[1];
    auto result = Tensor::create({1}, prediction->requires_grad);
    auto stats = std::make_shared<wm::DeviceVector>((size_t)rows * WM_CE_STATS);
    ck(wm_cross_entropy_fwd(prediction->data.dev(), target->data.dev(), rows, cols, stats->dev_write(),
                            result->data.dev_write()),
       "CrossEntropyLoss");
    if (result->requires_grad) {
        Tensor* res = result.get();
        auto pred = prediction;
        result->parents = {pred};
        result->grad_fn = [pred, target, res, stats, rows, cols]() {
            int acc = 0;
            float* gx = grad_target(pred, &acc);
            ck(wm_cross_entropy_bwd(pred->data.dev(), target->data.dev(), stats->dev(), res->grad.dev(), gx, acc,
                                    rows, cols),
               "CrossEntropyLoss backward");
        };
    }
    return result;
}

// loss.cpp:99-127: a gather, and a scatter into the prediction's gradient.
TensorPtr NLLLoss::forward(const TensorPtr& prediction, const TensorPtr& target) {
    check_head(prediction, target, "NLLLoss");
    const int64_t rows = (int64_t)prediction->shape[0], cols = (int64_t)prediction->shape[1];
    auto result = Tensor::create({1}, prediction->requires_grad);
    ck(wm_nll_fwd(prediction->data.dev(), target->data.dev(), rows, cols, result->data.dev_write()), "NLLLoss");
    if (result->requires_grad) {
        Tensor* res = result.get();
        auto pred = prediction;
        result->parents = {pred};
        result->grad_fn = [pred, target, res, rows, cols]() {
            int acc = 0;
            float* gx = grad_target(pred, &acc);
            ck(wm_nll_bwd(target->data.dev(), res->grad.dev(), gx, acc, rows, cols), "NLLLoss backward");
        };
    }
    return result;
}

// loss.cpp:260-331: softmax statistics, the label's focal term and the
// closure's per-row factors in one row pass; one streaming backward pass.
TensorPtr FocalLoss::forward(const TensorPtr& prediction, const TensorPtr& target) {
    check_head(prediction, target, "FocalLoss");
    const int64_t rows = (int64_t)prediction->shape[0], cols = (int64_t)prediction->shape[1];
    auto result = Tensor::create({1}, prediction->requires_grad);
    auto stats = std::make_shared<wm::DeviceVector>((size_t)rows * WM_FOCAL_STATS);
    ck(wm_focal_fwd(prediction->data.dev(), target->data.dev(), rows, cols, gamma, alpha, stats->dev_write(),
                    result->data.dev_write()),
       "FocalLoss");
    if (result->requires_grad) {
        Tensor* res = result.get();
        auto pred = prediction;
        const float g = gamma, a = alpha;
        result->parents = {pred};
        result->grad_fn = [pred, target, res, stats, rows, cols, g, a]() {
            int acc = 0;
            float* gx = grad_target(pred, &acc);
            ck(wm_focal_bwd(pred->data.dev(), target->data.dev(), stats->dev(), res->grad.dev(), gx, acc, rows, cols,
                            g, a),
               "FocalLoss backward");
        };
    }
    return result;
}
