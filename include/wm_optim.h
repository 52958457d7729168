/*
 * wm_optim.h -- C ABI of libwm_hip's parameter-update kernels: the optimizer
 * steps, gradient clipping and gradient unscaling of whitematter's training
 * loop (reference core/optimizer.cpp, core/amp.h), next to the Tensor path of
 * wm_hip.h.
 *
 * The reference updates parameters with host loops over each parameter's
 * std::vector<float> data and grad and keeps the optimizer state (velocity,
 * first/second moments) in host vectors.  Here parameters, gradients and
 * state stay in HBM and each update is one streaming pass.  The drop-in C++
 * optimizer classes (whitematter_amd/core/optimizer.{h,cpp}) call these
 * entry points from step(), clip_grad_norm_() and friends.
 *
 * Conventions are those of wm_hip.h (status codes, wm_last_error(), device
 * pointers, one library stream).  Every update computes exactly the float
 * expression of the reference loop it names, in the same operation order,
 * with IEEE division and square root and no contraction into fused
 * multiply-adds, so results equal a strict IEEE evaluation of the reference
 * source bit for bit.  Updates are in place (p, state and g may not alias
 * each other).
 */
#ifndef WM_OPTIM_H
#define WM_OPTIM_H

#include <stddef.h>
#include <stdint.h>

#ifdef __cplusplus
extern "C" {
#endif

/* SGD::step, core/optimizer.cpp:22-36.  velocity may be NULL when
 * momentum == 0 (the reference keeps no velocity then):
 *   momentum > 0:  v = momentum * v + g;  p -= lr * v
 *   otherwise:     p -= lr * g                                            */
int wm_sgd_step(float* p, const float* g, float* velocity, int64_t n, float lr, float momentum);

/* Adam::step, core/optimizer.cpp:46-66, one parameter tensor; the caller
 * increments t and passes bias_correction{1,2} = 1 - beta{1,2}^t computed
 * as the reference does (float(1.0 - pow(double(beta), t))):
 *   m = b1 m + (1 - b1) g;  v = b2 v + (1 - b2) g g
 *   p -= lr * (m / bc1) / (sqrt(v / bc2) + eps)                            */
int wm_adam_step(float* p, const float* g, float* m, float* v, int64_t n, float lr, float beta1, float beta2,
                 float eps, float bias_correction1, float bias_correction2);

/* AdamW::step, core/optimizer.cpp:76-100 (decoupled weight decay):
 *   p -= lr * ((m / bc1) / (sqrt(v / bc2) + eps) + weight_decay * p)       */
int wm_adamw_step(float* p, const float* g, float* m, float* v, int64_t n, float lr, float beta1, float beta2,
                  float eps, float bias_correction1, float bias_correction2, float weight_decay);

/* RMSprop::step, core/optimizer.cpp:112-138.  buffer may be NULL when
 * momentum == 0.  g is not modified (the weight-decayed gradient is local):
 *   g' = g + weight_decay * p   (only when weight_decay != 0)
 *   v = alpha v + (1 - alpha) g' g';  avg = sqrt(v) + eps
 *   momentum > 0:  buf = momentum * buf + g' / avg;  p -= lr * buf
 *   otherwise:     p -= lr * g' / avg                                      */
int wm_rmsprop_step(float* p, const float* g, float* v, float* buffer, int64_t n, float lr, float alpha, float eps,
                    float momentum, float weight_decay);

/* get_grad_norm's accumulation, core/optimizer.cpp:145-153: *total (one
 * device float) += sum of g[i]^2 over this tensor.  The tensor's sum is a
 * fixed-order tree and is added to *total on the device in call order, so a
 * sequence of calls is deterministic; the reference's sequential float sum is
 * matched to the sum tolerance, not bit for bit. */
int wm_grad_sumsq_accumulate(const float* g, int64_t n, float* total);

/* clip_grad_norm_'s scaling, core/optimizer.cpp:155-164, with the norm read
 * on the device (no host round trip):
 *   clip_coef = max_norm / (sqrt(*total_sumsq) + 1e-6f);
 *   if (clip_coef < 1) g[i] *= clip_coef                                   */
int wm_clip_grad_norm_scale(float* g, int64_t n, const float* total_sumsq, float max_norm);

/* clip_grad_value_, core/optimizer.cpp:166-177:
 *   g > c -> c;  g < -c -> -c;  otherwise (NaN included) unchanged         */
int wm_clip_grad_value(float* g, int64_t n, float clip_value);

/* GradScaler::unscale, core/amp.h:125-147, over a list of gradient tensors
 * (host arrays of `count` device pointers and sizes, in the optimizer's
 * parameter order; NULL or size-0 entries are skipped like an empty grad).
 * Walks the tensors in order multiplying each element by inv_scale and stops
 * at the first element whose product is not finite: tensors before it are
 * fully unscaled, its own tensor up to (not including) that element, the
 * rest untouched -- the reference's early break.  *found_inf (host) is set to
 * 1 if such an element exists, else 0.  One search launch over the whole list
 * and one scaling launch; synchronises with the library stream in between
 * (the stopping position decides what is written). */
int wm_grad_unscale(int count, float* const* grads, const int64_t* sizes, float inv_scale, int* found_inf);

/* check_gradients_finite, core/amp.h:293-300: *all_finite (host) = 1 when
 * every element of every listed gradient is finite, else 0.  Read-only: one
 * search launch over the list (and its finalize), then one synchronisation
 * for the answer. */
int wm_grads_finite_multi(int count, const float* const* g, const int64_t* n, int* all_finite);

/* ---- multi-tensor variants ----------------------------------------------
 * The same updates over a whole parameter list in one launch: host arrays of
 * `count` device pointers (one per parameter tensor) and sizes; zero-size
 * entries are skipped.  Each element gets exactly the single-tensor update,
 * so results equal calling the single-tensor entry point per tensor in list
 * order -- also when entries share arrays (a parameter listed twice): the
 * list is cut into runs whose written arrays overlap nothing else in the
 * run, one launch per run, in list order.  The list's descriptor table is uploaded on the library stream
 * through pinned staging; the call does not wait for the GPU.  This is what
 * the drop-in optimizers' step() uses: a model's many small parameter tensors
 * would otherwise cost one kernel launch each.                             */
int wm_sgd_step_multi(int count, float* const* p, const float* const* g, float* const* velocity, const int64_t* n,
                      float lr, float momentum);
int wm_adam_step_multi(int count, float* const* p, const float* const* g, float* const* m, float* const* v,
                       const int64_t* n, float lr, float beta1, float beta2, float eps, float bias_correction1,
                       float bias_correction2);
int wm_adamw_step_multi(int count, float* const* p, const float* const* g, float* const* m, float* const* v,
                        const int64_t* n, float lr, float beta1, float beta2, float eps, float bias_correction1,
                        float bias_correction2, float weight_decay);
int wm_rmsprop_step_multi(int count, float* const* p, const float* const* g, float* const* v, float* const* buffer,
                          const int64_t* n, float lr, float alpha, float eps, float momentum, float weight_decay);

/* get_grad_norm's sum of squares over a gradient list: *total (device) =
 * sum over every element of every tensor, a fixed-order two-pass sum.      */
int wm_grad_sumsq_multi(int count, const float* const* g, const int64_t* n, float* total);
/* clip_grad_norm_amp's sum of squares, core/amp.h:303-312: sum of (g * mul)^2
 * with each element scaled before it is squared (mul = 1 / scale), so still-
 * scaled gradients do not overflow the sum the way g^2 * mul^2 would. */
int wm_grad_sumsq_scaled_multi(int count, const float* const* g, const int64_t* n, float mul, float* total);

/* clip_grad_norm_'s scaling and clip_grad_value_ over a gradient list.      */
int wm_clip_grad_norm_scale_multi(int count, float* const* g, const int64_t* n, const float* total_sumsq,
                                  float max_norm);
int wm_clip_grad_value_multi(int count, float* const* g, const int64_t* n, float clip_value);

/* ---- deferred gradient scaling -------------------------------------------
 * GradScaler::unscale (core/amp.h:125-147) and clip_grad_norm_
 * (core/optimizer.cpp:155-164) multiply every gradient in place; done eagerly
 * that is a read and a write of each gradient after the pass that decides the
 * factor (the first non-finite position, the norm).  The drop-in records the
 * multiplication with the gradient instead and lets the next pass over the
 * gradients apply it as it reads them -- the optimizer step, a norm, a
 * finiteness search -- or writes it once (wm_grad_scale_apply_multi) before
 * any other use.  A gradient's stored values g and its wm_grad_scale give its
 * values as the reference holds them:
 *   v = g[i];
 *   if (i < unscale_count) v = v * unscale;           (unscale's prefix)
 *   if (clip_sumsq) { c = clip_max_norm / (sqrt(*clip_sumsq) + 1e-6f);
 *                     if (c < 1) v = v * c; }         (clip_grad_norm_)
 * each product rounded to fp32 as the reference's in-place multiply is, so
 * every result below equals the eager passes' bit for bit.  clip_sumsq is a
 * device float (the norm's sum of squares), read when the scaling is
 * applied.  No counterpart in the reference (its multiplications are
 * eager); these entry points take one wm_grad_scale per list entry.        */
typedef struct wm_grad_scale {
    float unscale;           /* factor of the elements [0, unscale_count) */
    int64_t unscale_count;   /* 0: no deferred unscale; at most the tensor's size */
    const float* clip_sumsq; /* NULL: no deferred clip */
    float clip_max_norm;
} wm_grad_scale;

/* Write each gradient's deferred scaling into it (g[i] = v).                */
int wm_grad_scale_apply_multi(int count, float* const* g, const wm_grad_scale* gs, const int64_t* n);
/* The optimizer steps above on the gradients' values v (their stored values
 * and deferred scalings, gs may be NULL: none).                             */
int wm_sgd_step_multi_gs(int count, float* const* p, const float* const* g, const wm_grad_scale* gs,
                         float* const* velocity, const int64_t* n, float lr, float momentum);
int wm_adam_step_multi_gs(int count, float* const* p, const float* const* g, const wm_grad_scale* gs,
                          float* const* m, float* const* v, const int64_t* n, float lr, float beta1, float beta2,
                          float eps, float bias_correction1, float bias_correction2);
int wm_adamw_step_multi_gs(int count, float* const* p, const float* const* g, const wm_grad_scale* gs,
                           float* const* m, float* const* v, const int64_t* n, float lr, float beta1, float beta2,
                           float eps, float bias_correction1, float bias_correction2, float weight_decay);
int wm_rmsprop_step_multi_gs(int count, float* const* p, const float* const* g, const wm_grad_scale* gs,
                             float* const* v, float* const* buffer, const int64_t* n, float lr, float alpha,
                             float eps, float momentum, float weight_decay);
/* *total (device) = sum over the list of (v * mul)^2 (get_grad_norm,
 * clip_grad_norm_amp).                                                      */
int wm_grad_sumsq_multi_gs(int count, const float* const* g, const wm_grad_scale* gs, const int64_t* n, float mul,
                           float* total);
/* where[0], where[1] (host) = list position and element of the first value
 * v with v * scale not finite, in list order, or (count, 0): unscale's stop
 * (scale = 1 / loss scale) and check_gradients_finite (scale = 1).  Read-only;
 * synchronises for the answer.                                              */
int wm_grad_first_bad_multi_gs(int count, const float* const* g, const wm_grad_scale* gs, const int64_t* n,
                               float scale, int64_t* where);

#ifdef __cplusplus
}
#endif

#endif /* WM_OPTIM_H */
