// device_vector.h -- host/device-coherent fp32 storage with std::vector's API.
//
// The reference keeps Tensor::data and Tensor::grad as std::vector<float>
// (core/tensor.h:35-36) and its callers touch them directly: size(), data(),
// begin()/end(), operator[], resize(), empty(), whole-vector assignment from
// std::vector<float> or an initializer list, range-for.  DeviceVector keeps
// that surface so callers compile unchanged, while the authoritative copy of
// the values lives in device memory (libwm_hip's pool):
//
//   host access   const access copies device -> host if the host mirror is
//                 stale; non-const access (which may write) also marks the
//                 device copy stale, so the next kernel re-uploads it;
//   device access dev() uploads a stale device copy; dev_write() hands out the
//                 buffer for a full overwrite (no upload) and marks the host
//                 mirror stale; dev_rw() does both;
//   known zero    a fresh zero-filled vector (a new gradient, zero_grad) is
//                 only a flag: nothing is allocated or filled until someone
//                 needs the values, and the first backward contribution can
//                 overwrite instead of read-modify-write (dev_accum()).
//   deferred scaling  GradScaler::unscale and clip_grad_norm_ multiply a
//                 gradient in place; the drop-in records the multiplication
//                 instead (defer_unscale / defer_clip, include/wm_optim.h's
//                 wm_grad_scale) and the next pass over the gradient applies
//                 it as it reads: the optimizer step, a norm or a finiteness
//                 search take dev_deferred().  Every other access sees the
//                 scaled values: host access, dev(), dev_rw() and dev_accum()
//                 first write the scaling into the device copy (one pass);
//                 a full overwrite, set_zero() or fill() drop it.
//
// Not thread-safe, like the reference Tensor.
#pragma once

#include <cstddef>
#include <cstdint>
#include <initializer_list>
#include <memory>
#include <vector>

#include "wm_optim.h"

namespace wm {

class DeviceVector {
public:
    using value_type = float;
    using size_type = std::size_t;
    using iterator = float*;
    using const_iterator = const float*;
    using reference = float&;
    using const_reference = const float&;

    DeviceVector() = default;
    explicit DeviceVector(size_type n, float value = 0.0f);
    DeviceVector(const std::vector<float>& v);  // NOLINT: implicit, like a vector copy
    DeviceVector(std::initializer_list<float> v);
    template <class It>
    DeviceVector(It first, It last) : DeviceVector(std::vector<float>(first, last)) {}
    DeviceVector(const DeviceVector& o);
    DeviceVector(DeviceVector&& o) noexcept;
    ~DeviceVector();

    DeviceVector& operator=(const DeviceVector& o);
    DeviceVector& operator=(DeviceVector&& o) noexcept;
    DeviceVector& operator=(const std::vector<float>& v);
    DeviceVector& operator=(std::initializer_list<float> v);

    // ---- std::vector surface (host side, coherent) ------------------------
    size_type size() const { return n_; }
    bool empty() const { return n_ == 0; }
    float* data();
    const float* data() const;
    float& operator[](size_type i) { return data()[i]; }
    const float& operator[](size_type i) const { return data()[i]; }
    float& at(size_type i);
    const float& at(size_type i) const;
    float& front() { return data()[0]; }
    float& back() { return data()[n_ - 1]; }
    iterator begin() { return data(); }
    iterator end() { return data() + n_; }
    const_iterator begin() const { return data(); }
    const_iterator end() const { return data() + n_; }
    const_iterator cbegin() const { return data(); }
    const_iterator cend() const { return data() + n_; }
    void resize(size_type n, float value = 0.0f);
    void assign(size_type n, float value);
    template <class It>
    void assign(It first, It last) { *this = std::vector<float>(first, last); }
    void clear();
    void push_back(float v);
    operator std::vector<float>() const;  // NOLINT: implicit, copies to the host
    bool operator==(const DeviceVector& o) const;
    bool operator!=(const DeviceVector& o) const { return !(*this == o); }

    // ---- device side -------------------------------------------------------
    // Device pointer to current values (uploads / zero-fills as needed).
    const float* dev() const;
    // Device pointer for a full overwrite: no upload, host mirror goes stale.
    float* dev_write();
    // Device pointer for read-modify-write.
    float* dev_rw();
    // Pointer for a gradient contribution: *accumulate = 0 when the buffer is
    // known to be zero (the kernel then overwrites it), 1 otherwise.
    float* dev_accum(int* accumulate);
    // Mark the contents as all zeros without touching memory.
    void set_zero();
    bool known_zero() const { return zero_; }
    // Fill with a constant on the device.
    void fill(float value);

    // ---- deferred scaling (gradients) ------------------------------------
    // Record v[i] *= factor for i < count (GradScaler::unscale's prefix).  An
    // earlier deferred scaling is written first.
    void defer_unscale(float factor, int64_t count);
    // Record clip_grad_norm_'s v[i] *= c, c = max_norm / (sqrt(*sumsq) + 1e-6f),
    // applied when c < 1; sumsq is a one-element device vector kept alive
    // until the scaling is applied.  An earlier deferred clip is written
    // first (an unscale may stay: the clip follows it).
    void defer_clip(std::shared_ptr<const DeviceVector> sumsq, float max_norm);
    bool deferred() const { return def_count_ > 0 || def_sumsq_ != nullptr; }
    // Device pointer to the stored values and, in *gs, the scaling that gives
    // the current values from them (none: unscale_count 0, clip_sumsq NULL).
    const float* dev_deferred(wm_grad_scale* gs) const;
    // Write a deferred scaling into the device copy.
    void apply_deferred() const;

private:
    void ensure_dev_alloc() const;
    void sync_host() const;   // make the host mirror current
    void release();
    void drop_deferred() const;
    const float* dev_stored() const;  // current device copy of the stored values (no deferred scaling applied)

    size_type n_ = 0;
    mutable float* d_ = nullptr;           // device buffer (capacity n_), lazily allocated
    mutable std::vector<float> h_;         // host mirror
    mutable bool host_valid_ = true;       // h_ holds the current values
    mutable bool dev_valid_ = true;        // d_ holds the current values
    bool zero_ = false;                    // logically all zeros (neither copy needs to be valid)
    // deferred scaling of the device copy (the host mirror is stale while one is set)
    mutable float def_unscale_ = 1.0f;
    mutable int64_t def_count_ = 0;
    mutable std::shared_ptr<const DeviceVector> def_sumsq_;
    mutable float def_max_norm_ = 0.0f;
};

// fp16 bit patterns (uint16_t) with std::vector<uint16_t>'s API and the
// same coherence rules as DeviceVector (no known-zero state): the storage of
// HalfTensor::data (core/amp.h:258), so fp16 tensors stay in HBM and
// converting them to fp32 is one device pass.
class HalfVector {
public:
    using value_type = uint16_t;
    using size_type = std::size_t;
    using iterator = uint16_t*;
    using const_iterator = const uint16_t*;

    HalfVector() = default;
    explicit HalfVector(size_type n);  // n zeros, as std::vector<uint16_t>(n)
    // Device storage of n elements whose contents are unset until the caller
    // overwrites all of them through dev_write() (HalfTensor's converting
    // constructor does, at once).
    static HalfVector uninitialized(size_type n);
    HalfVector(const std::vector<uint16_t>& v);  // NOLINT: implicit, like a vector copy
    HalfVector(const HalfVector& o);
    HalfVector(HalfVector&& o) noexcept;
    ~HalfVector();
    HalfVector& operator=(const HalfVector& o);
    HalfVector& operator=(HalfVector&& o) noexcept;
    HalfVector& operator=(const std::vector<uint16_t>& v);

    size_type size() const { return n_; }
    bool empty() const { return n_ == 0; }
    uint16_t* data();
    const uint16_t* data() const;
    uint16_t& operator[](size_type i) { return data()[i]; }
    const uint16_t& operator[](size_type i) const { return data()[i]; }
    iterator begin() { return data(); }
    iterator end() { return data() + n_; }
    const_iterator begin() const { return data(); }
    const_iterator end() const { return data() + n_; }
    void resize(size_type n, uint16_t value = 0);
    void clear();
    operator std::vector<uint16_t>() const;  // NOLINT: implicit, copies to the host
    bool operator==(const HalfVector& o) const;

    // Device pointer to current values (uploads a stale device copy).
    const uint16_t* dev() const;
    // Device pointer for a full overwrite: no upload, host mirror goes stale.
    uint16_t* dev_write();

private:
    void ensure_dev_alloc() const;
    void sync_host() const;
    void release();

    size_type n_ = 0;
    mutable uint16_t* d_ = nullptr;
    mutable std::vector<uint16_t> h_;
    mutable bool host_valid_ = true;
    mutable bool dev_valid_ = true;
};

}  // namespace wm
