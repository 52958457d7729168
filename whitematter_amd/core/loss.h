// loss.h -- drop-in for whitematter's core/loss.h with every loss computed on
// the GPU.
//
// Same classes, members, constructors, defaults and include guard as the
// reference header (core/loss.h:1-76), so code written against it compiles
// unchanged.  The bodies (loss.cpp) call the device entry points of
// include/wm_loss.h, or compose device Tensor ops where the reference does
// (MSELoss, L1Loss); the loss value stays in HBM until someone reads it.
#ifndef LOSS_H
#define LOSS_H

#include "tensor.h"

class LossFunction {
public:
    virtual ~LossFunction() = default;
    virtual TensorPtr forward(const TensorPtr& prediction, const TensorPtr& target) = 0;

    TensorPtr operator()(const TensorPtr& prediction, const TensorPtr& target) { return forward(prediction, target); }
};

class MSELoss : public LossFunction {
public:
    TensorPtr forward(const TensorPtr& prediction, const TensorPtr& target) override;
};

class L1Loss : public LossFunction {
public:
    TensorPtr forward(const TensorPtr& prediction, const TensorPtr& target) override;
};

class SmoothL1Loss : public LossFunction {
public:
    float beta;  // |x| below beta: quadratic; above: linear
    SmoothL1Loss(float beta = 1.0f) : beta(beta) {}
    TensorPtr forward(const TensorPtr& prediction, const TensorPtr& target) override;
};

class CrossEntropyLoss : public LossFunction {
public:
    TensorPtr forward(const TensorPtr& prediction, const TensorPtr& target) override;
};

class NLLLoss : public LossFunction {
public:
    TensorPtr forward(const TensorPtr& prediction, const TensorPtr& target) override;
};

class BCELoss : public LossFunction {
public:
    TensorPtr forward(const TensorPtr& prediction, const TensorPtr& target) override;
};

class BCEWithLogitsLoss : public LossFunction {
public:
    TensorPtr forward(const TensorPtr& prediction, const TensorPtr& target) override;
};

class KLDivLoss : public LossFunction {
public:
    bool log_target;  // target holds log-probabilities
    KLDivLoss(bool log_target = false) : log_target(log_target) {}
    TensorPtr forward(const TensorPtr& prediction, const TensorPtr& target) override;
};

class FocalLoss : public LossFunction {
public:
    float alpha;  // class weight; negative: none
    float gamma;  // focusing exponent
    FocalLoss(float gamma = 2.0f, float alpha = -1.0f) : alpha(alpha), gamma(gamma) {}
    TensorPtr forward(const TensorPtr& prediction, const TensorPtr& target) override;
};

class BinaryFocalLoss : public LossFunction {
public:
    float alpha;  // weight of the positive class; negative: none
    float gamma;  // focusing exponent
    BinaryFocalLoss(float gamma = 2.0f, float alpha = 0.25f) : alpha(alpha), gamma(gamma) {}
    TensorPtr forward(const TensorPtr& prediction, const TensorPtr& target) override;
};

#endif  // LOSS_H
