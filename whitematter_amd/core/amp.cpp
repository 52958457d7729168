// amp.cpp -- the device parts of the drop-in amp.h: HalfTensor's
// conversions, GradScaler::unscale, check_gradients_finite and
// clip_grad_norm_amp (reference core/amp.h:125-147, :256-286, :293-327),
// through libwm_hip's C ABI.
#include "amp.h"

#include <cmath>
#include <limits>
#include <stdexcept>
#include <string>

#include "wm_hip.h"
#include "wm_optim.h"

namespace {

void check(int rc, const char* what) {
    if (rc != WM_OK) throw std::runtime_error(std::string("whitematter_amd ") + what + ": " + wm_last_error());
}

// The gradients that hold values: a gradient that is empty or known to be
// all zeros is skipped (scaling zeros by a finite factor leaves zeros, and
// zeros are finite).  `write` hands out pointers for in-place updates (the
// host mirrors go stale), otherwise read-only ones.
void live_grads(const std::vector<TensorPtr>& params, std::vector<float*>& ptrs, std::vector<int64_t>& sizes,
                bool write = true) {
    for (const auto& p : params) {
        if (!p || p->grad.empty() || p->grad.known_zero()) continue;
        ptrs.push_back(write ? p->grad.dev_rw() : const_cast<float*>(p->grad.dev()));
        sizes.push_back((int64_t)p->grad.size());
    }
}

// Whether any listed parameter has a non-empty gradient (known-zero ones
// included).
bool any_grad(const std::vector<TensorPtr>& params) {
    for (const auto& p : params)
        if (p && !p->grad.empty()) return true;
    return false;
}

}  // namespace

// core/amp.h:125-147
bool GradScaler::unscale(Optimizer* optimizer) {
    if (!enabled_) return true;
    const float inv_scale = 1.0f / scale_;
    if (!std::isfinite(inv_scale)) {
        // Every product is then non-finite, zeros included (0 * inf, x * NaN):
        // the reference stops at the first element of the first non-empty
        // gradient, having changed nothing.
        found_inf_or_nan_ = any_grad(optimizer->params);
        return !found_inf_or_nan_;
    }
    std::vector<float*> ptrs;
    std::vector<int64_t> sizes;
    live_grads(optimizer->params, ptrs, sizes);
    int found = 0;
    check(wm_grad_unscale((int)ptrs.size(), ptrs.data(), sizes.data(), inv_scale, &found), "GradScaler::unscale");
    found_inf_or_nan_ = found != 0;
    return !found_inf_or_nan_;
}

// core/amp.h:263-267
HalfTensor::HalfTensor(const TensorPtr& tensor) : shape(tensor->shape) {
    const size_t n = tensor->data.size();
    data = wm::HalfVector::uninitialized(n);  // every element is written below
    if (n == 0) return;
    check(wm_f32_to_f16_rtz(data.dev_write(), tensor->data.dev(), (int64_t)n), "HalfTensor");
}

// core/amp.h:270-274
TensorPtr HalfTensor::to_float(bool requires_grad) const {
    auto result = Tensor::create(shape, requires_grad);
    if (result->data.size() != data.size()) result->data.resize(data.size());
    if (data.empty()) return result;
    check(wm_f16_to_f32(result->data.dev_write(), data.dev(), (int64_t)data.size()), "HalfTensor::to_float");
    return result;
}

// core/amp.h:293-300: every element finite; a read-only device search.
bool check_gradients_finite(const std::vector<TensorPtr>& params) {
    std::vector<float*> ptrs;
    std::vector<int64_t> sizes;
    live_grads(params, ptrs, sizes, false);
    int all = 1;
    check(wm_grads_finite_multi((int)ptrs.size(), const_cast<const float* const*>(ptrs.data()), sizes.data(), &all),
          "check_gradients_finite");
    return all != 0;
}

// core/amp.h:303-327: norm of g / scale over all gradients; when
// max_norm / (norm + 1e-6f) < 1 every gradient (still scaled) is multiplied
// by that coefficient.
float clip_grad_norm_amp(const std::vector<TensorPtr>& params, float max_norm, float scale) {
    const float inv_scale = 1.0f / scale;
    std::vector<float*> ptrs;
    std::vector<int64_t> sizes;
    live_grads(params, ptrs, sizes);
    float sumsq = 0.0f;
    if (!ptrs.empty()) {
        void* d = nullptr;
        check(wm_alloc(&d, sizeof(float)), "clip_grad_norm_amp");
        int rc = wm_fill(static_cast<float*>(d), 0.0f, 1);
        if (rc == WM_OK)
            rc = wm_grad_sumsq_scaled_multi((int)ptrs.size(), const_cast<const float* const*>(ptrs.data()),
                                            sizes.data(), inv_scale, static_cast<float*>(d));
        if (rc == WM_OK) rc = wm_d2h(&sumsq, d, sizeof(float));
        wm_free(d);
        check(rc, "clip_grad_norm_amp");
    }
    // Known-zero gradients were skipped; with a non-finite inv_scale their
    // zeros would add 0 * inf (or 0 * NaN) = NaN to the reference's sum.
    if (!std::isfinite(inv_scale))
        for (const auto& p : params)
            if (p && !p->grad.empty() && p->grad.known_zero()) sumsq = std::numeric_limits<float>::quiet_NaN();
    // each element scaled before it is squared, as the reference does
    const float total_norm = std::sqrt(sumsq);
    const float clip_coef = max_norm / (total_norm + 1e-6f);
    if (clip_coef < 1.0f)
        for (size_t k = 0; k < ptrs.size(); ++k)
            check(wm_unary(WM_SCALE, ptrs[k], ptrs[k], sizes[k], clip_coef, 0.0f), "clip_grad_norm_amp");
    return total_norm;
}
