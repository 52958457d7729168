/*
 * wm_loss.h -- C ABI of libwm_hip's loss heads: whitematter's loss functions
 * (reference core/loss.h, core/loss.cpp) on the device, next to the Tensor
 * path of wm_hip.h.
 *
 * The reference computes every loss with host loops over the prediction's
 * and target's std::vector<float> data; CrossEntropyLoss and FocalLoss first
 * run log_softmax / softmax over the whole [batch, classes] prediction and
 * then gather the label entries on the host.  Here the classification heads
 * are one fused row pass each: the row statistics of (log_)softmax and the
 * label gather happen in the same kernel, nothing of size batch x classes is
 * written by the forward, and the backward recomputes the probabilities from
 * the logits and the saved per-row statistics in one streaming pass.  The
 * batch mean is a fixed-order two-level sum on the device, so the loss is
 * deterministic and never leaves HBM.  The drop-in loss classes
 * (whitematter_amd/core/loss.{h,cpp}) call these entry points.
 *
 * Conventions are those of wm_hip.h (status codes, wm_last_error(), device
 * pointers, one library stream, `accumulate` = 1 for "+=", 0 when the
 * gradient buffer is known to be zero).  `loss` is one device float;
 * `loss_grad` is the device float holding d(out)/d(loss) (the loss tensor's
 * grad[0]); each backward computes scale = *loss_grad / denominator on the
 * device as the reference closures do.
 *
 * Labels are fp32 class indices, read as the reference reads them:
 * static_cast<size_t>(target->data[i]) (core/loss.cpp:80), i.e. truncated
 * toward zero.  A label that does not truncate to a class in [0, classes)
 * (negative, too large, NaN) -- an out-of-bounds access in the reference --
 * makes that row's loss term NaN, so the loss is NaN; the classification
 * heads' backward writes NaN over that row (cross entropy, focal) or skips it
 * (NLL, which has no position to write).
 */
#ifndef WM_LOSS_H
#define WM_LOSS_H

#include <stddef.h>
#include <stdint.h>

#ifdef __cplusplus
extern "C" {
#endif

/* Floats of per-row statistics each fused head saves for its backward.     */
#define WM_CE_STATS 2
#define WM_FOCAL_STATS 8

/* CrossEntropyLoss::forward, core/loss.cpp:67-97, fused with the
 * log_softmax it calls (core/tensor.cpp:1593-1616):
 *   log_sum_r = max_r + log(sum_j exp(x_rj - max_r))
 *   *loss = -(sum_r (x_r,label_r - log_sum_r)) / rows
 * logits [rows, classes], labels [rows].  stats [rows * WM_CE_STATS] receives
 * {log_sum_r, x_r,label_r - log_sum_r} per row.  The label term equals the
 * entry wm_log_softmax_fwd writes at that position, bit for bit.          */
int wm_cross_entropy_fwd(const float* logits, const float* labels, int64_t rows, int64_t classes, float* stats,
                         float* loss);

/* The backward of that loss and of its log_softmax in one pass (closures at
 * core/loss.cpp:86-93 and core/tensor.cpp:1621-1632):
 *   scale = *loss_grad / rows;  g_rj = (0 - scale) at the label, else 0
 *   grad_rj (+)= g_rj - exp(x_rj - log_sum_r) * (0 - scale)
 * which is the log_softmax closure applied to the label scatter, element for
 * element the same arithmetic.                                              */
int wm_cross_entropy_bwd(const float* logits, const float* labels, const float* stats, const float* loss_grad,
                         float* grad, int accumulate, int64_t rows, int64_t classes);

/* NLLLoss::forward, core/loss.cpp:99-127: *loss = -(sum_r pred_r,label_r) / rows. */
int wm_nll_fwd(const float* pred, const float* labels, int64_t rows, int64_t classes, float* loss);

/* NLLLoss's closure: grad_r,label_r -= *loss_grad / rows.  With accumulate = 0
 * the whole [rows, classes] buffer is written (zeros and the label entries). */
int wm_nll_bwd(const float* labels, const float* loss_grad, float* grad, int accumulate, int64_t rows,
               int64_t classes);

/* FocalLoss::forward, core/loss.cpp:260-294, fused with its softmax
 * (core/tensor.cpp:1548-1572):
 *   p_rj = exp(x_rj - max_r) / sum_j exp(x_rj - max_r)
 *   p_t = max(p_r,label, 1e-7);  l_r = -(1 - p_t)^gamma * log(p_t)  (* alpha if alpha >= 0)
 *   *loss = (sum_r l_r) / rows
 * stats [rows * WM_FOCAL_STATS] receives the row's max and 1/sum, the three
 * per-row factors of the closure and l_r.                                   */
int wm_focal_fwd(const float* logits, const float* labels, int64_t rows, int64_t classes, float gamma, float alpha,
                 float* stats, float* loss);

/* FocalLoss's closure, core/loss.cpp:296-328, with the probabilities
 * recomputed from the logits and the saved statistics:
 *   label:  g = p_c * (gamma log(p_t) (1-p_t)^gamma - (1-p_t)^gamma) + (1-p_t)^gamma
 *   other:  g = -p_c * ((1-p_t)^(gamma-1) * (gamma p_t log(p_t) + (1-p_t)))
 *   g *= alpha (alpha >= 0);  grad_rc (+)= (*loss_grad / rows) * g         */
int wm_focal_bwd(const float* logits, const float* labels, const float* stats, const float* loss_grad, float* grad,
                 int accumulate, int64_t rows, int64_t classes, float gamma, float alpha);

/* The element-wise losses whose reference bodies are host loops, one term and
 * one gradient per element of pred / target (n elements each):            */
enum wm_pointwise_loss {
    WM_L_SMOOTH_L1 = 0,     /* SmoothL1Loss, core/loss.cpp:21-65; p0 = beta          */
    WM_L_BCE = 1,           /* BCELoss, :130-164                                      */
    WM_L_BCE_LOGITS = 2,    /* BCEWithLogitsLoss, :166-202                            */
    WM_L_KLDIV = 3,         /* KLDivLoss, :204-258, target as probabilities           */
    WM_L_KLDIV_LOG = 4,     /* KLDivLoss with log_target = true                       */
    WM_L_BINARY_FOCAL = 5   /* BinaryFocalLoss, :333-418; p0 = gamma, p1 = alpha      */
};

/* *loss = (sum_i term_i) / denom, the reference's loop and final division:
 * denom is n for every kind except the KL divergence, whose reference divides
 * by the batch size (prediction->shape[0]).                                */
int wm_pointwise_loss_fwd(int kind, const float* pred, const float* target, int64_t n, float p0, float p1,
                          float denom, float* loss);

/* grad_i (+)= (*loss_grad / denom) * d term_i / d pred_i, the reference closure. */
int wm_pointwise_loss_bwd(int kind, const float* pred, const float* target, int64_t n, float p0, float p1,
                          float denom, const float* loss_grad, float* grad, int accumulate);

#ifdef __cplusplus
}
#endif

#endif /* WM_LOSS_H */
