// amp.cpp -- the device parts of the drop-in amp.h: HalfTensor's
// conversions, GradScaler::unscale, check_gradients_finite and
// clip_grad_norm_amp (reference core/amp.h:125-147, :256-286, :293-327),
// through libwm_hip's C ABI.
#include "amp.h"

#include <cmath>
#include <limits>
#include <memory>
#include <stdexcept>
#include <string>

#include "wm_hip.h"
#include "wm_optim.h"

namespace {

void check(int rc, const char* what) {
    if (rc != WM_OK) throw std::runtime_error(std::string("whitematter_amd ") + what + ": " + wm_last_error());
}

// The gradients that hold values, with their deferred scalings: a gradient
// that is empty is skipped, and one known to be all zeros unless `zeros`
// (scaling +0 by a positive finite factor leaves +0, and zeros are finite;
// a negative factor would make them -0).  `vecs` gets the storage of each;
// the pointers are for read-only passes that apply the deferred scalings as
// they read.
void live_grads_deferred(const std::vector<TensorPtr>& params, std::vector<wm::DeviceVector*>& vecs,
                         std::vector<const float*>& ptrs, std::vector<wm_grad_scale>& gs,
                         std::vector<int64_t>& sizes, bool zeros = false) {
    for (const auto& p : params) {
        if (!p || p->grad.empty() || (!zeros && p->grad.known_zero())) continue;
        vecs.push_back(&p->grad);
        gs.emplace_back();
        ptrs.push_back(p->grad.dev_deferred(&gs.back()));
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
    std::vector<wm::DeviceVector*> vecs;
    std::vector<const float*> ptrs;
    std::vector<wm_grad_scale> gs;
    std::vector<int64_t> sizes;
    live_grads_deferred(optimizer->params, vecs, ptrs, gs, sizes, inv_scale < 0.0f);
    bool listed_twice = false;
    for (size_t i = 0; i < vecs.size() && !listed_twice; ++i)
        for (size_t j = i + 1; j < vecs.size(); ++j)
            if (vecs[i] == vecs[j]) { listed_twice = true; break; }
    if (listed_twice) {
        // A gradient listed twice is scaled twice, the second pass searching
        // the first pass's products: the eager search-and-scale runs per list
        // position in order (wm_grad_unscale).
        std::vector<float*> rw;
        for (auto* v : vecs) rw.push_back(v->dev_rw());
        int found = 0;
        check(wm_grad_unscale((int)rw.size(), rw.data(), sizes.data(), inv_scale, &found), "GradScaler::unscale");
        found_inf_or_nan_ = found != 0;
        return !found_inf_or_nan_;
    }
    // One read of every gradient finds the stop; the products themselves are
    // deferred (DeviceVector::defer_unscale) to the pass that reads the
    // gradients next -- normally the optimizer step.
    int64_t where[2] = {0, 0};
    check(wm_grad_first_bad_multi_gs((int)ptrs.size(), ptrs.data(), gs.data(), sizes.data(), inv_scale, where),
          "GradScaler::unscale");
    const int64_t stop = where[0];
    for (size_t k = 0; k < vecs.size(); ++k) {
        const int64_t cnt = (int64_t)k < stop ? sizes[k] : ((int64_t)k == stop ? where[1] : 0);
        vecs[k]->defer_unscale(inv_scale, cnt);
    }
    found_inf_or_nan_ = stop < (int64_t)vecs.size();
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
    std::vector<wm::DeviceVector*> vecs;
    std::vector<const float*> ptrs;
    std::vector<wm_grad_scale> gs;
    std::vector<int64_t> sizes;
    live_grads_deferred(params, vecs, ptrs, gs, sizes);
    int64_t where[2] = {0, 0};
    check(wm_grad_first_bad_multi_gs((int)ptrs.size(), ptrs.data(), gs.data(), sizes.data(), 1.0f, where),
          "check_gradients_finite");
    return where[0] >= (int64_t)ptrs.size();
}

// core/amp.h:303-327: norm of g / scale over all gradients; when
// max_norm / (norm + 1e-6f) < 1 every gradient (still scaled) is multiplied
// by that coefficient.
float clip_grad_norm_amp(const std::vector<TensorPtr>& params, float max_norm, float scale) {
    const float inv_scale = 1.0f / scale;
    std::vector<wm::DeviceVector*> vecs;
    std::vector<const float*> ptrs;
    std::vector<wm_grad_scale> gs;
    std::vector<int64_t> sizes;
    live_grads_deferred(params, vecs, ptrs, gs, sizes);
    float sumsq = 0.0f;
    auto total = std::make_shared<wm::DeviceVector>(1, 0.0f);
    if (!ptrs.empty()) {
        check(wm_grad_sumsq_multi_gs((int)ptrs.size(), ptrs.data(), gs.data(), sizes.data(), inv_scale,
                                     total->dev_write()),
              "clip_grad_norm_amp");
        sumsq = (*total)[0];
    }
    // Known-zero gradients were skipped; with a non-finite inv_scale their
    // zeros would add 0 * inf (or 0 * NaN) = NaN to the reference's sum.
    if (!std::isfinite(inv_scale))
        for (const auto& p : params)
            if (p && !p->grad.empty() && p->grad.known_zero()) sumsq = std::numeric_limits<float>::quiet_NaN();
    // each element scaled before it is squared, as the reference does
    const float total_norm = std::sqrt(sumsq);
    const float clip_coef = max_norm / (total_norm + 1e-6f);
    // Deferred like clip_grad_norm_'s: the device recomputes this coefficient
    // from the same sum of squares, bit for bit, when the products are taken.
    if (clip_coef < 1.0f)  // every listing of every gradient, as the reference's loop (known-zero ones too)
        for (const auto& p : params)
            if (p && !p->grad.empty()) p->grad.defer_clip(total, max_norm);
    return total_norm;
}
