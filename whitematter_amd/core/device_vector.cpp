// device_vector.cpp -- see device_vector.h.
#include "device_vector.h"

#include <algorithm>
#include <cmath>
#include <cstring>
#include <stdexcept>
#include <string>

#include "wm_hip.h"

namespace wm {

namespace {

void ck(int rc, const char* what) {
    if (rc != WM_OK) throw std::runtime_error(std::string(what) + ": " + wm_last_error());
}

}  // namespace

DeviceVector::DeviceVector(size_type n, float value) : n_(n) {
    if (n_ == 0) return;
    if (value == 0.0f && !std::signbit(value)) set_zero();
    else fill(value);
}

DeviceVector::DeviceVector(const std::vector<float>& v) : n_(v.size()), h_(v) {
    host_valid_ = true;
    dev_valid_ = false;
}

DeviceVector::DeviceVector(std::initializer_list<float> v) : DeviceVector(std::vector<float>(v)) {}

DeviceVector::DeviceVector(const DeviceVector& o) : n_(o.n_) {
    if (n_ == 0) return;
    if (o.zero_) {
        set_zero();
    } else if (o.dev_valid_) {
        ensure_dev_alloc();
        ck(wm_d2d(d_, o.d_, n_ * sizeof(float)), "DeviceVector copy");
        dev_valid_ = true;
        host_valid_ = false;
        // the copy holds the same stored values: it takes the same scaling
        def_unscale_ = o.def_unscale_;
        def_count_ = o.def_count_;
        def_sumsq_ = o.def_sumsq_;
        def_max_norm_ = o.def_max_norm_;
    } else {
        h_ = o.h_;
        host_valid_ = true;
        dev_valid_ = false;
    }
}

DeviceVector::DeviceVector(DeviceVector&& o) noexcept
    : n_(o.n_), d_(o.d_), h_(std::move(o.h_)), host_valid_(o.host_valid_), dev_valid_(o.dev_valid_), zero_(o.zero_),
      def_unscale_(o.def_unscale_), def_count_(o.def_count_), def_sumsq_(std::move(o.def_sumsq_)),
      def_max_norm_(o.def_max_norm_) {
    o.n_ = 0;
    o.d_ = nullptr;
    o.host_valid_ = o.dev_valid_ = true;
    o.zero_ = false;
    o.drop_deferred();
}

DeviceVector::~DeviceVector() { release(); }

DeviceVector& DeviceVector::operator=(const DeviceVector& o) {
    if (this == &o) return *this;
    if (o.n_ == n_ && n_ > 0 && d_ && !o.zero_ && o.dev_valid_) {
        // same size: copy into this buffer, as std::vector's copy assignment
        // reuses its storage (a gradient assigned every step keeps its address)
        ck(wm_d2d(d_, o.d_, n_ * sizeof(float)), "DeviceVector copy");
        dev_valid_ = true;
        host_valid_ = false;
        zero_ = false;
        def_unscale_ = o.def_unscale_;
        def_count_ = o.def_count_;
        def_sumsq_ = o.def_sumsq_;
        def_max_norm_ = o.def_max_norm_;
        return *this;
    }
    DeviceVector tmp(o);
    *this = std::move(tmp);
    return *this;
}

DeviceVector& DeviceVector::operator=(DeviceVector&& o) noexcept {
    if (this == &o) return *this;
    release();
    n_ = o.n_;
    d_ = o.d_;
    h_ = std::move(o.h_);
    host_valid_ = o.host_valid_;
    dev_valid_ = o.dev_valid_;
    zero_ = o.zero_;
    def_unscale_ = o.def_unscale_;
    def_count_ = o.def_count_;
    def_sumsq_ = std::move(o.def_sumsq_);
    def_max_norm_ = o.def_max_norm_;
    o.n_ = 0;
    o.d_ = nullptr;
    o.host_valid_ = o.dev_valid_ = true;
    o.zero_ = false;
    o.drop_deferred();
    return *this;
}

DeviceVector& DeviceVector::operator=(const std::vector<float>& v) {
    release();
    drop_deferred();
    n_ = v.size();
    h_ = v;
    host_valid_ = true;
    dev_valid_ = false;
    zero_ = false;
    return *this;
}

DeviceVector& DeviceVector::operator=(std::initializer_list<float> v) { return *this = std::vector<float>(v); }

void DeviceVector::release() {
    if (d_) {
        wm_free(d_);
        d_ = nullptr;
    }
}

void DeviceVector::ensure_dev_alloc() const {
    if (d_ || n_ == 0) return;
    void* p = nullptr;
    ck(wm_alloc(&p, n_ * sizeof(float)), "DeviceVector allocation");
    d_ = static_cast<float*>(p);
}

void DeviceVector::sync_host() const {
    if (n_ == 0) return;
    if (host_valid_) return;
    apply_deferred();
    if (zero_) {
        h_.assign(n_, 0.0f);
    } else {
        h_.resize(n_);
        ck(wm_d2h(h_.data(), d_, n_ * sizeof(float)), "DeviceVector device->host");
    }
    host_valid_ = true;
}

const float* DeviceVector::data() const {
    if (n_ == 0) return h_.data();
    sync_host();
    return h_.data();
}

float* DeviceVector::data() {
    if (n_ == 0) return h_.data();
    sync_host();
    // The caller may write through the pointer: the host copy becomes the
    // only valid one.
    zero_ = false;
    dev_valid_ = false;
    return h_.data();
}

float& DeviceVector::at(size_type i) {
    if (i >= n_) throw std::out_of_range("DeviceVector::at");
    return data()[i];
}

const float& DeviceVector::at(size_type i) const {
    if (i >= n_) throw std::out_of_range("DeviceVector::at");
    return data()[i];
}

const float* DeviceVector::dev() const {
    if (n_ == 0) return nullptr;
    apply_deferred();
    return dev_stored();
}

const float* DeviceVector::dev_stored() const {
    ensure_dev_alloc();
    if (!dev_valid_) {
        if (zero_) {
            ck(wm_fill(d_, 0.0f, (int64_t)n_), "DeviceVector zero fill");
        } else {
            ck(wm_h2d(d_, h_.data(), n_ * sizeof(float)), "DeviceVector host->device");
        }
        dev_valid_ = true;
    }
    return d_;
}

float* DeviceVector::dev_write() {
    if (n_ == 0) return nullptr;
    drop_deferred();
    ensure_dev_alloc();
    zero_ = false;
    dev_valid_ = true;
    host_valid_ = false;
    return d_;
}

float* DeviceVector::dev_rw() {
    if (n_ == 0) return nullptr;
    dev();
    zero_ = false;
    host_valid_ = false;
    return d_;
}

float* DeviceVector::dev_accum(int* accumulate) {
    if (zero_) {
        *accumulate = 0;
        return dev_write();
    }
    *accumulate = 1;
    return dev_rw();
}

void DeviceVector::set_zero() {
    drop_deferred();
    zero_ = n_ > 0;
    host_valid_ = n_ == 0;
    dev_valid_ = n_ == 0;
}

void DeviceVector::fill(float value) {
    if (n_ == 0) return;
    if (value == 0.0f && !std::signbit(value)) {
        set_zero();
        return;
    }
    drop_deferred();
    ensure_dev_alloc();
    ck(wm_fill(d_, value, (int64_t)n_), "DeviceVector fill");
    zero_ = false;
    dev_valid_ = true;
    host_valid_ = false;
}

void DeviceVector::resize(size_type n, float value) {
    if (n == n_) return;
    if (n_ == 0 || (zero_ && value == 0.0f && !std::signbit(value))) {
        release();
        drop_deferred();
        h_.clear();
        n_ = n;
        if (value == 0.0f && !std::signbit(value)) set_zero();
        else fill(value);
        return;
    }
    sync_host();
    h_.resize(n, value);
    release();
    n_ = n;
    zero_ = false;
    host_valid_ = true;
    dev_valid_ = false;
}

void DeviceVector::assign(size_type n, float value) {
    release();
    drop_deferred();
    h_.clear();
    n_ = n;
    zero_ = false;
    host_valid_ = dev_valid_ = true;
    if (n_ == 0) return;
    if (value == 0.0f && !std::signbit(value)) set_zero();
    else fill(value);
}

void DeviceVector::clear() {
    release();
    drop_deferred();
    h_.clear();
    n_ = 0;
    zero_ = false;
    host_valid_ = dev_valid_ = true;
}

void DeviceVector::push_back(float v) {
    sync_host();
    h_.push_back(v);
    release();
    ++n_;
    zero_ = false;
    host_valid_ = true;
    dev_valid_ = false;
}

DeviceVector::operator std::vector<float>() const {
    sync_host();
    return std::vector<float>(h_.begin(), h_.begin() + (std::ptrdiff_t)n_);
}

bool DeviceVector::operator==(const DeviceVector& o) const {
    if (n_ != o.n_) return false;
    if (n_ == 0) return true;
    // Element-wise ==, as std::vector<float> compares (NaN != NaN, -0 == +0).
    const float* a = data();
    const float* b = o.data();
    return std::equal(a, a + n_, b);
}

// ---- deferred scaling --------------------------------------------------------

void DeviceVector::drop_deferred() const {
    def_unscale_ = 1.0f;
    def_count_ = 0;
    def_sumsq_.reset();
    def_max_norm_ = 0.0f;
}

void DeviceVector::apply_deferred() const {
    if (!deferred()) return;
    // Hold the sum of squares until the kernel that reads it is enqueued: the
    // call allocates its descriptor table from the pool, which must not hand
    // out the sum's block before that.
    const std::shared_ptr<const DeviceVector> keep = def_sumsq_;
    wm_grad_scale gs{def_unscale_, def_count_, keep ? keep->dev() : nullptr, def_max_norm_};
    float* p = d_;
    const int64_t n = (int64_t)n_;
    drop_deferred();
    ck(wm_grad_scale_apply_multi(1, &p, &gs, &n), "deferred gradient scaling");
}

void DeviceVector::defer_unscale(float factor, int64_t count) {
    if (n_ == 0 || count <= 0) return;
    // zeros times a positive finite factor stay +0; any other factor makes
    // them -0 or NaN, so the zeros are written out first
    if (zero_ && factor > 0.0f && std::isfinite(factor)) return;
    if (count > (int64_t)n_) count = (int64_t)n_;
    if (deferred()) apply_deferred();
    dev_stored();
    zero_ = false;
    host_valid_ = false;
    def_unscale_ = factor;
    def_count_ = count;
}

void DeviceVector::defer_clip(std::shared_ptr<const DeviceVector> sumsq, float max_norm) {
    if (n_ == 0 || !sumsq) return;
    // a max_norm >= 0 gives a coefficient >= 0 (or NaN, not applied): zeros
    // stay +0; a negative or infinite one makes them -0 or NaN
    if (zero_ && max_norm >= 0.0f && std::isfinite(max_norm)) return;
    if (def_sumsq_) apply_deferred();
    dev_stored();  // an unscale deferred before stays: the clip follows it
    zero_ = false;
    host_valid_ = false;
    def_sumsq_ = std::move(sumsq);
    def_max_norm_ = max_norm;
}

const float* DeviceVector::dev_deferred(wm_grad_scale* gs) const {
    wm_grad_scale none{1.0f, 0, nullptr, 0.0f};
    if (!deferred()) {
        *gs = none;
        return dev();
    }
    *gs = wm_grad_scale{def_unscale_, def_count_, def_sumsq_ ? def_sumsq_->dev() : nullptr, def_max_norm_};
    return d_;  // valid: a scaling is only deferred on a current device copy
}

// ---- HalfVector -----------------------------------------------------------

// Zeros in the host mirror, uploaded when the device first needs them.
HalfVector::HalfVector(size_type n) : n_(n), h_(n, 0) { dev_valid_ = n_ == 0; }

HalfVector HalfVector::uninitialized(size_type n) {
    HalfVector v;
    v.n_ = n;
    if (n == 0) return v;
    v.ensure_dev_alloc();
    v.host_valid_ = false;  // neither copy holds values until the caller's write
    v.dev_valid_ = true;
    return v;
}

HalfVector::HalfVector(const std::vector<uint16_t>& v) : n_(v.size()), h_(v) { dev_valid_ = n_ == 0; }

HalfVector::HalfVector(const HalfVector& o) : n_(o.n_) {
    if (n_ == 0) return;
    if (o.dev_valid_) {
        ensure_dev_alloc();
        ck(wm_d2d(d_, o.d_, n_ * sizeof(uint16_t)), "HalfVector copy");
        host_valid_ = false;
    } else {
        h_ = o.h_;
        dev_valid_ = false;
    }
}

HalfVector::HalfVector(HalfVector&& o) noexcept
    : n_(o.n_), d_(o.d_), h_(std::move(o.h_)), host_valid_(o.host_valid_), dev_valid_(o.dev_valid_) {
    o.n_ = 0;
    o.d_ = nullptr;
    o.host_valid_ = o.dev_valid_ = true;
}

HalfVector::~HalfVector() { release(); }

HalfVector& HalfVector::operator=(const HalfVector& o) {
    if (this == &o) return *this;
    HalfVector tmp(o);
    return *this = std::move(tmp);
}

HalfVector& HalfVector::operator=(HalfVector&& o) noexcept {
    if (this == &o) return *this;
    release();
    n_ = o.n_;
    d_ = o.d_;
    h_ = std::move(o.h_);
    host_valid_ = o.host_valid_;
    dev_valid_ = o.dev_valid_;
    o.n_ = 0;
    o.d_ = nullptr;
    o.host_valid_ = o.dev_valid_ = true;
    return *this;
}

HalfVector& HalfVector::operator=(const std::vector<uint16_t>& v) { return *this = HalfVector(v); }

void HalfVector::release() {
    if (d_) {
        wm_free(d_);
        d_ = nullptr;
    }
}

void HalfVector::ensure_dev_alloc() const {
    if (d_ || n_ == 0) return;
    void* p = nullptr;
    ck(wm_alloc(&p, n_ * sizeof(uint16_t)), "HalfVector allocation");
    d_ = static_cast<uint16_t*>(p);
}

void HalfVector::sync_host() const {
    if (n_ == 0 || host_valid_) return;
    h_.resize(n_);
    ck(wm_d2h(h_.data(), d_, n_ * sizeof(uint16_t)), "HalfVector device->host");
    host_valid_ = true;
}

const uint16_t* HalfVector::data() const {
    sync_host();
    return h_.data();
}

uint16_t* HalfVector::data() {
    sync_host();
    dev_valid_ = n_ == 0;  // the caller may write through the pointer
    return h_.data();
}

const uint16_t* HalfVector::dev() const {
    if (n_ == 0) return nullptr;
    ensure_dev_alloc();
    if (!dev_valid_) {
        ck(wm_h2d(d_, h_.data(), n_ * sizeof(uint16_t)), "HalfVector host->device");
        dev_valid_ = true;
    }
    return d_;
}

uint16_t* HalfVector::dev_write() {
    if (n_ == 0) return nullptr;
    ensure_dev_alloc();
    dev_valid_ = true;
    host_valid_ = false;
    return d_;
}

void HalfVector::resize(size_type n, uint16_t value) {
    if (n == n_) return;
    sync_host();
    h_.resize(n, value);
    release();
    n_ = n;
    host_valid_ = true;
    dev_valid_ = n_ == 0;
}

void HalfVector::clear() {
    release();
    h_.clear();
    n_ = 0;
    host_valid_ = dev_valid_ = true;
}

HalfVector::operator std::vector<uint16_t>() const {
    sync_host();
    return std::vector<uint16_t>(h_.begin(), h_.begin() + (std::ptrdiff_t)n_);
}

bool HalfVector::operator==(const HalfVector& o) const {
    if (n_ != o.n_) return false;
    if (n_ == 0) return true;
    const uint16_t* a = data();
    const uint16_t* b = o.data();
    return std::equal(a, a + n_, b);
}

}  // namespace wm
