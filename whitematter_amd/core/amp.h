// amp.h -- drop-in for the reference's core/amp.h (same classes, functions,
// signatures, defaults and AMP_H guard), with the storage conversions and the
// gradient scans on the device.
//
//   float_to_half / half_to_float / to_half / from_half   (:15-90)
//       host conversions with the reference's bit formulas: fp32 -> fp16 by
//       truncation (round toward zero; |x| >= 65536 -> inf; a NaN keeps the
//       top ten payload bits, so a payload only in the low 13 bits becomes
//       inf), fp16 -> fp32 exact.
//   HalfTensor (:256-286)
//       the conversion runs on the device (wm_f32_to_f16_rtz /
//       wm_f16_to_f32, the same formulas) and the halves stay in HBM:
//       `data` is a wm::HalfVector with std::vector<uint16_t>'s API, whose
//       host copy is made only when a caller reads it.
//   GradScaler (:96-204)
//       unscale() (wm_grad_unscale) has the reference's semantics:
//       gradients are multiplied by 1 / scale in parameter order up to the
//       first product that is not finite, which and everything after it stay
//       as they were.  On the device that is a read-only search for that
//       first product, a 16-byte copy of its position to the host, then one
//       scaling pass over what precedes it.
//   AmpContext, AutocastGuard (:210-250)   host state, unchanged.
//   check_gradients_finite, clip_grad_norm_amp (:293-327)
//       check_gradients_finite is one read-only device search (no
//       gradient is written); clip_grad_norm_amp is one sum-of-squares pass
//       over g / scale and, when it clips, one scaling pass.  Only the flag
//       or the norm crosses to the host.
#ifndef AMP_H
#define AMP_H

#include "optimizer.h"
#include "tensor.h"

#include <algorithm>
#include <cstdint>
#include <cstring>
#include <vector>

// =============================================================================
// Half-precision (fp16) storage conversions
// =============================================================================

inline uint16_t float_to_half(float f) {
    uint32_t x;
    std::memcpy(&x, &f, sizeof x);
    const uint32_t sign = (x >> 16) & 0x8000u;
    const int32_t e = (int32_t)((x >> 23) & 0xFFu) - 112;  // fp16 biased exponent
    const uint32_t m = x & 0x7FFFFFu;
    if (e == 143) return (uint16_t)(sign | 0x7C00u | (m >> 13));  // inf / NaN (payload truncated)
    if (e > 30) return (uint16_t)(sign | 0x7C00u);                // overflow
    if (e > 0) return (uint16_t)(sign | ((uint32_t)e << 10) | (m >> 13));
    if (e < -10) return (uint16_t)sign;                            // below half the smallest subnormal
    return (uint16_t)(sign | (((m | 0x800000u) >> (1 - e)) >> 13));  // subnormal half, truncated
}

inline float half_to_float(uint16_t h) {
    const uint32_t sign = (uint32_t)(h & 0x8000u) << 16;
    const uint32_t e = (h >> 10) & 0x1Fu;
    uint32_t m = h & 0x3FFu;
    uint32_t bits;
    if (e == 31) {
        bits = sign | 0x7F800000u | (m << 13);
    } else if (e != 0) {
        bits = sign | ((e + 112) << 23) | (m << 13);
    } else if (m == 0) {
        bits = sign;
    } else {
        // subnormal half: normalise into an fp32 normal
        int32_t ee = 113;
        while (!(m & 0x400u)) {
            m <<= 1;
            --ee;
        }
        bits = sign | ((uint32_t)ee << 23) | ((m & 0x3FFu) << 13);
    }
    float f;
    std::memcpy(&f, &bits, sizeof f);
    return f;
}

inline std::vector<uint16_t> to_half(const std::vector<float>& data) {
    std::vector<uint16_t> out(data.size());
    for (size_t i = 0; i < data.size(); i++) out[i] = float_to_half(data[i]);
    return out;
}

inline std::vector<float> from_half(const std::vector<uint16_t>& half_data) {
    std::vector<float> out(half_data.size());
    for (size_t i = 0; i < half_data.size(); i++) out[i] = half_to_float(half_data[i]);
    return out;
}

// =============================================================================
// GradScaler
// =============================================================================

class GradScaler {
public:
    GradScaler(float init_scale = 65536.0f, float growth_factor = 2.0f, float backoff_factor = 0.5f,
               int growth_interval = 2000, bool enabled = true)
        : scale_(init_scale),
          growth_factor_(growth_factor),
          backoff_factor_(backoff_factor),
          growth_interval_(growth_interval),
          growth_tracker_(0),
          enabled_(enabled) {}

    float get_scale() const { return enabled_ ? scale_ : 1.0f; }
    bool is_enabled() const { return enabled_; }

    TensorPtr scale(const TensorPtr& loss) const { return enabled_ ? loss->mul(scale_) : loss; }

    // Multiplies every gradient by 1 / scale on the device; false (and no
    // further scaling) from the first product that is not finite.
    bool unscale(Optimizer* optimizer);

    void step(Optimizer* optimizer, bool already_unscaled = false) {
        if (!enabled_) {
            optimizer->step();
            return;
        }
        if (!already_unscaled) unscale(optimizer);
        if (!found_inf_or_nan_) optimizer->step();
    }

    void update() {
        if (!enabled_) return;
        if (found_inf_or_nan_) {
            scale_ *= backoff_factor_;
            growth_tracker_ = 0;
        } else if (++growth_tracker_ >= growth_interval_) {
            scale_ *= growth_factor_;
            growth_tracker_ = 0;
        }
        scale_ = std::max(1.0f, std::min(scale_, 65536.0f * 65536.0f));  // a NaN scale becomes 1
        found_inf_or_nan_ = false;
    }

    float scale() const { return scale_; }
    int growth_tracker() const { return growth_tracker_; }
    void set_scale(float s) { scale_ = s; }
    void set_growth_tracker(int t) { growth_tracker_ = t; }

private:
    float scale_;
    float growth_factor_;
    float backoff_factor_;
    int growth_interval_;
    int growth_tracker_;
    bool enabled_;
    bool found_inf_or_nan_ = false;
};

// =============================================================================
// AmpContext / AutocastGuard
// =============================================================================

class AmpContext {
public:
    static AmpContext& instance() {
        static AmpContext ctx;
        return ctx;
    }
    void set_enabled(bool enabled) { enabled_ = enabled; }
    bool is_enabled() const { return enabled_; }
    enum class Dtype { Float32, Float16, BFloat16 };
    void set_dtype(Dtype dtype) { dtype_ = dtype; }
    Dtype get_dtype() const { return dtype_; }

private:
    AmpContext() : enabled_(false), dtype_(Dtype::Float16) {}
    bool enabled_;
    Dtype dtype_;
};

class AutocastGuard {
public:
    AutocastGuard(bool enabled = true, AmpContext::Dtype dtype = AmpContext::Dtype::Float16)
        : prev_enabled_(AmpContext::instance().is_enabled()), prev_dtype_(AmpContext::instance().get_dtype()) {
        AmpContext::instance().set_enabled(enabled);
        AmpContext::instance().set_dtype(dtype);
    }
    ~AutocastGuard() {
        AmpContext::instance().set_enabled(prev_enabled_);
        AmpContext::instance().set_dtype(prev_dtype_);
    }

private:
    bool prev_enabled_;
    AmpContext::Dtype prev_dtype_;
};

// =============================================================================
// HalfTensor: fp16 storage of a tensor
// =============================================================================

class HalfTensor {
public:
    // The fp16 bits live in HBM; wm::HalfVector keeps std::vector<uint16_t>'s
    // API (size(), data(), operator[], conversion to std::vector) for callers.
    wm::HalfVector data;
    std::vector<size_t> shape;

    HalfTensor() = default;

    // Truncating fp16 copy of tensor->data, converted on the device.
    explicit HalfTensor(const TensorPtr& tensor);

    // A new tensor of `shape` holding the exact fp32 values of `data`
    // (converted on the device).
    TensorPtr to_float(bool requires_grad = false) const;

    size_t size() const {
        size_t s = 1;
        for (auto d : shape) s *= d;
        return s;
    }

    size_t memory_saved() const { return size() * sizeof(float) - size() * sizeof(uint16_t); }
};

// =============================================================================
// Mixed precision training utilities
// =============================================================================

// True when every gradient element is finite (a read-only device search).
bool check_gradients_finite(const std::vector<TensorPtr>& params);

// Global norm of the gradients divided by `scale`; when max_norm / (norm +
// 1e-6) < 1 every gradient is multiplied by that coefficient.  Returns the
// norm.  On the device; the sum of squares is a sum (fp32 tolerance, not
// the reference's sequential order).
float clip_grad_norm_amp(const std::vector<TensorPtr>& params, float max_norm, float scale = 1.0f);

#endif  // AMP_H
