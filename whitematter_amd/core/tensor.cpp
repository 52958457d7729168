// tensor.cpp -- whitematter's Tensor on MI355X: the elementwise / broadcast /
// reduction / softmax ops and their backward closures, each a call into the
// C ABI of libwm_hip (include/wm_hip.h).  Shape rules, tracking rules and the
// autograd engine follow the reference's core/tensor.cpp line by line where
// they are observable (cited per function); the loops themselves are gone.
#include "tensor.h"

#include <algorithm>
#include <cstdint>
#include <stdexcept>
#include <string>

#include "wm_gemm.h"
#include "wm_hip.h"

namespace {

void ck(int rc, const char* what) {
    if (rc != WM_OK) throw std::runtime_error(std::string("whitematter_amd ") + what + ": " + wm_last_error());
}

size_t numel_of(const std::vector<size_t>& s) {
    size_t n = 1;
    for (auto d : s) n *= d;
    return n;
}

std::vector<int64_t> i64(const std::vector<size_t>& s) { return std::vector<int64_t>(s.begin(), s.end()); }

// A gradient buffer sized like the tensor's data (the reference allocates it
// at creation when requires_grad is set, core/tensor.cpp:413,418).
float* grad_target(const TensorPtr& t, int* accumulate) {
    if (t->grad.size() != t->data.size()) t->grad = wm::DeviceVector(t->data.size());
    return t->grad.dev_accum(accumulate);
}

// Device int64 buffer for saved max/min positions.
std::shared_ptr<int64_t> device_index_buffer(size_t n) {
    void* p = nullptr;
    ck(wm_alloc(&p, std::max<size_t>(n, 1) * sizeof(int64_t)), "index buffer");
    return std::shared_ptr<int64_t>(static_cast<int64_t*>(p), [](int64_t* q) { wm_free(q); });
}

[[noreturn]] void out_of_scope(const char* what) {
    throw std::logic_error(std::string("Tensor::") + what +
                           ": not part of the MI355X elementwise/broadcast/reduction build");
}

bool needs_input(int op) {
    return op == WM_RELU || op == WM_LOG || op == WM_POWS || op == WM_ABS || op == WM_CLAMP;
}
bool needs_output(int op) { return op == WM_SIGMOID || op == WM_TANH || op == WM_EXP || op == WM_SQRT; }

}  // namespace

// ---------------------------------------------------------------------------
// GradMode (core/tensor.cpp:26-42)
// ---------------------------------------------------------------------------

bool GradMode::enabled_ = true;

bool GradMode::is_enabled() { return enabled_; }
void GradMode::set_enabled(bool enabled) { enabled_ = enabled; }

NoGradGuard::NoGradGuard() : prev_mode_(GradMode::is_enabled()) { GradMode::set_enabled(false); }
NoGradGuard::~NoGradGuard() { GradMode::set_enabled(prev_mode_); }

// ---------------------------------------------------------------------------
// Storage and factories (core/tensor.cpp:404-454)
// ---------------------------------------------------------------------------

static std::mt19937 rng(42);

Tensor::Tensor() : requires_grad(false) {}

// A new tensor is zero-filled (reference :408-414); here "zero" is a flag on
// the storage until someone needs the values.
Tensor::Tensor(const std::vector<size_t>& shape, bool requires_grad)
    : data(numel_of(shape)), shape(shape), requires_grad(requires_grad) {
    if (requires_grad) grad = wm::DeviceVector(data.size());
}

Tensor::Tensor(const std::vector<float>& data, const std::vector<size_t>& shape, bool requires_grad)
    : data(data), shape(shape), requires_grad(requires_grad) {
    if (requires_grad) grad = wm::DeviceVector(this->data.size());
}

TensorPtr Tensor::create(const std::vector<size_t>& shape, bool requires_grad) {
    return std::make_shared<Tensor>(shape, requires_grad);
}

TensorPtr Tensor::create(const std::vector<float>& data, const std::vector<size_t>& shape, bool requires_grad) {
    return std::make_shared<Tensor>(data, shape, requires_grad);
}

TensorPtr Tensor::zeros(const std::vector<size_t>& shape, bool requires_grad) { return create(shape, requires_grad); }

TensorPtr Tensor::ones(const std::vector<size_t>& shape, bool requires_grad) {
    auto t = create(shape, requires_grad);
    t->data.fill(1.0f);
    return t;
}

// Same generator and distribution as the reference (:404, :441-446), so the
// values match it on the same standard library.
TensorPtr Tensor::randn(const std::vector<size_t>& shape, bool requires_grad) {
    std::vector<float> v(numel_of(shape));
    std::normal_distribution<float> dist(0.0f, 1.0f);
    for (auto& x : v) x = dist(rng);
    return create(v, shape, requires_grad);
}

TensorPtr Tensor::xavier(size_t fan_in, size_t fan_out, bool requires_grad) {
    std::vector<float> v(fan_in * fan_out);
    float std = std::sqrt(2.0f / (fan_in + fan_out));
    std::normal_distribution<float> dist(0.0f, std);
    for (auto& x : v) x = dist(rng);
    return create(v, {fan_in, fan_out}, requires_grad);
}

TensorPtr Tensor::concat(const std::vector<TensorPtr>&, int) { out_of_scope("concat"); }
TensorPtr Tensor::stack(const std::vector<TensorPtr>&, int) { out_of_scope("stack"); }

size_t Tensor::size() const { return data.size(); }
size_t Tensor::ndim() const { return shape.size(); }

float Tensor::item() const {
    assert(data.size() == 1);
    return data[0];
}

// zero_grad (:725-727) fills with zeros; the flag is equivalent.
void Tensor::zero_grad() { grad.set_zero(); }

float& Tensor::operator[](size_t idx) { return data[idx]; }
float Tensor::operator[](size_t idx) const { return data[idx]; }

float& Tensor::at(const std::vector<size_t>& indices) {
    size_t idx = 0, stride = 1;
    for (int i = (int)shape.size() - 1; i >= 0; i--) {
        idx += indices[i] * stride;
        stride *= shape[i];
    }
    return data[idx];
}

float Tensor::at(const std::vector<size_t>& indices) const {
    size_t idx = 0, stride = 1;
    for (int i = (int)shape.size() - 1; i >= 0; i--) {
        idx += indices[i] * stride;
        stride *= shape[i];
    }
    return data[idx];
}

// ---------------------------------------------------------------------------
// Autograd engine (core/tensor.cpp:750-781)
// ---------------------------------------------------------------------------

bool Tensor::should_track_grad() const { return requires_grad && GradMode::is_enabled(); }

void Tensor::build_topo(std::vector<Tensor*>& topo, std::vector<Tensor*>& visited) {
    if (std::find(visited.begin(), visited.end(), this) != visited.end()) return;
    visited.push_back(this);
    for (auto& p : parents) p->build_topo(topo, visited);
    topo.push_back(this);
}

// Root gradient overwritten with 1 (not accumulated), closures run in reverse
// topological order, then the graph is cleared (:763-781).
void Tensor::backward() {
    assert(data.size() == 1);
    if (grad.empty()) grad.resize(1, 0.0f);
    grad[0] = 1.0f;

    std::vector<Tensor*> topo, visited;
    build_topo(topo, visited);
    for (auto it = topo.rbegin(); it != topo.rend(); ++it) {
        if ((*it)->grad_fn) (*it)->grad_fn();
    }
    for (auto* t : topo) {
        t->grad_fn = nullptr;
        t->parents.clear();
    }
}

// ---------------------------------------------------------------------------
// Binary ops with broadcasting: add :897, sub :981, mul :1063, div :1147,
// pow(Tensor) :1385, max(Tensor) :1901, min(Tensor) :1986
// ---------------------------------------------------------------------------

TensorPtr Tensor::binary_op(int op, const TensorPtr& other) const {
    assert(shape.size() <= WM_MAX_DIMS && other->shape.size() <= WM_MAX_DIMS);
    const std::vector<int64_t> sa = i64(shape), sb = i64(other->shape);
    int64_t os[WM_MAX_DIMS];
    int on = 0;
    const int rc = wm_broadcast_shape(sa.data(), (int)sa.size(), sb.data(), (int)sb.size(), os, &on);
    assert(rc == WM_OK && "Shapes are not broadcastable");
    (void)rc;

    const bool track = (requires_grad || other->requires_grad) && GradMode::is_enabled();
    auto result = create(std::vector<size_t>(os, os + on), track);
    ck(wm_binary(op, result->data.dev_write(), data.dev(), sa.data(), (int)sa.size(), other->data.dev(), sb.data(),
                 (int)sb.size()),
       "binary op");

    if (track) {
        auto self_ptr = const_cast<Tensor*>(this)->shared_from_this();
        auto other_ptr = other;
        Tensor* res = result.get();  // the closure is owned by *res
        result->parents = {self_ptr, other_ptr};
        result->grad_fn = [self_ptr, other_ptr, res, op, sa, sb]() {
            const bool want_a = self_ptr->requires_grad, want_b = other_ptr->requires_grad;
            auto run = [&](bool a, bool b) {
                int acc_a = 0, acc_b = 0;
                float* ga = a ? grad_target(self_ptr, &acc_a) : nullptr;
                float* gb = b ? grad_target(other_ptr, &acc_b) : nullptr;
                // pow's d/db recomputes pow(a, b) on the device (out = NULL).
                ck(wm_binary_bwd(op, res->grad.dev(), self_ptr->data.dev(), sa.data(), (int)sa.size(),
                                 other_ptr->data.dev(), sb.data(), (int)sb.size(), nullptr, ga, acc_a, gb, acc_b),
                   "binary op backward");
            };
            if (want_a && want_b && self_ptr.get() == other_ptr.get()) {
                // x op x: both contributions go to the same buffer, one after the other.
                run(true, false);
                run(false, true);
            } else if (want_a || want_b) {
                run(want_a, want_b);
            }
        };
    }
    return result;
}

TensorPtr Tensor::add(const TensorPtr& other) const { return binary_op(WM_ADD, other); }
TensorPtr Tensor::sub(const TensorPtr& other) const { return binary_op(WM_SUB, other); }
TensorPtr Tensor::mul(const TensorPtr& other) const { return binary_op(WM_MUL, other); }
TensorPtr Tensor::div(const TensorPtr& other) const { return binary_op(WM_DIV, other); }
TensorPtr Tensor::pow(const TensorPtr& exponent) const { return binary_op(WM_POW, exponent); }
TensorPtr Tensor::max(const TensorPtr& other) const { return binary_op(WM_MAX, other); }
TensorPtr Tensor::min(const TensorPtr& other) const { return binary_op(WM_MIN, other); }

// ---------------------------------------------------------------------------
// Unary ops: mul(float) :1237, relu :1263, sigmoid :1281, tanh_ :1302,
// log_ :1323, exp_ :1343, pow(float) :1363, sqrt :1477, abs :1498, clamp :1524
// ---------------------------------------------------------------------------

TensorPtr Tensor::unary_op(int op, float p0, float p1) const {
    const bool track = requires_grad && GradMode::is_enabled();
    auto result = create(shape, track);
    const int64_t n = (int64_t)data.size();
    ck(wm_unary(op, result->data.dev_write(), data.dev(), n, p0, p1), "unary op");
    if (track) {
        auto self_ptr = const_cast<Tensor*>(this)->shared_from_this();
        Tensor* res = result.get();
        result->parents = {self_ptr};
        result->grad_fn = [self_ptr, res, op, p0, p1, n]() {
            int acc = 0;
            float* gx = grad_target(self_ptr, &acc);
            ck(wm_unary_bwd(op, res->grad.dev(), needs_input(op) ? self_ptr->data.dev() : nullptr,
                            needs_output(op) ? res->data.dev() : nullptr, gx, acc, n, p0, p1),
               "unary op backward");
        };
    }
    return result;
}

TensorPtr Tensor::mul(float scalar) const { return unary_op(WM_SCALE, scalar, 0.0f); }
// div(s) is mul(1/s) and neg() is mul(-1) in the reference (:1255-1261).
TensorPtr Tensor::div(float scalar) const { return mul(1.0f / scalar); }
TensorPtr Tensor::neg() const { return mul(-1.0f); }
TensorPtr Tensor::relu() const { return unary_op(WM_RELU, 0.0f, 0.0f); }
TensorPtr Tensor::sigmoid() const { return unary_op(WM_SIGMOID, 0.0f, 0.0f); }
TensorPtr Tensor::tanh_() const { return unary_op(WM_TANH, 0.0f, 0.0f); }
TensorPtr Tensor::log_() const { return unary_op(WM_LOG, 0.0f, 0.0f); }
TensorPtr Tensor::exp_() const { return unary_op(WM_EXP, 0.0f, 0.0f); }
TensorPtr Tensor::pow(float exponent) const { return unary_op(WM_POWS, exponent, 0.0f); }
TensorPtr Tensor::sqrt() const { return unary_op(WM_SQRT, 0.0f, 0.0f); }
TensorPtr Tensor::abs() const { return unary_op(WM_ABS, 0.0f, 0.0f); }
TensorPtr Tensor::clamp(float min_val, float max_val) const { return unary_op(WM_CLAMP, min_val, max_val); }

// ---------------------------------------------------------------------------
// Softmax / log_softmax (:1548, :1593): 2-D only, always the last axis
// ---------------------------------------------------------------------------

TensorPtr Tensor::softmax_op(bool log) const {
    assert(shape.size() == 2);
    const bool track = requires_grad && GradMode::is_enabled();
    auto result = create(shape, track);
    const int64_t rows = (int64_t)shape[0], cols = (int64_t)shape[1];
    ck((log ? wm_log_softmax_fwd : wm_softmax_fwd)(result->data.dev_write(), data.dev(), rows, cols), "softmax");
    if (track) {
        auto self_ptr = const_cast<Tensor*>(this)->shared_from_this();
        Tensor* res = result.get();
        result->parents = {self_ptr};
        result->grad_fn = [self_ptr, res, log, rows, cols]() {
            int acc = 0;
            float* gx = grad_target(self_ptr, &acc);
            ck((log ? wm_log_softmax_bwd : wm_softmax_bwd)(res->grad.dev(), res->data.dev(), gx, acc, rows, cols),
               "softmax backward");
        };
    }
    return result;
}

TensorPtr Tensor::softmax(int dim) const {
    if (dim < 0) dim = (int)shape.size() + dim;  // normalised, then unused (:1550)
    (void)dim;
    return softmax_op(false);
}

TensorPtr Tensor::log_softmax(int dim) const {
    if (dim < 0) dim = (int)shape.size() + dim;
    (void)dim;
    return softmax_op(true);
}

// ---------------------------------------------------------------------------
// Reductions: sum :1637, mean :1709, max(dim) :1723, min(dim) :1812,
// argmax :2075, argmin :2149
// ---------------------------------------------------------------------------

// sum/mean/max/min.  dim == -1 reduces everything; otherwise the tensor must
// be 2-D, dim 0 reduces rows and any other dim reduces columns.  For sum and
// mean the full reduction is shape [1] whatever keepdim says; for max/min
// keepdim keeps the rank (global_keep_rank).
TensorPtr Tensor::reduce_2d(int op, int dim, bool keepdim, bool global_keep_rank) const {
    std::vector<size_t> out_shape;
    int64_t outer, n, inner;
    if (dim == -1) {
        out_shape = (global_keep_rank && keepdim) ? std::vector<size_t>(shape.size(), 1) : std::vector<size_t>{1};
        outer = 1;
        n = (int64_t)data.size();
        inner = 1;
    } else {
        assert(shape.size() == 2);
        const size_t rows = shape[0], cols = shape[1];
        if (dim == 0) {
            out_shape = keepdim ? std::vector<size_t>{1, cols} : std::vector<size_t>{cols};
            outer = 1; n = (int64_t)rows; inner = (int64_t)cols;
        } else {
            out_shape = keepdim ? std::vector<size_t>{rows, 1} : std::vector<size_t>{rows};
            outer = (int64_t)rows; n = (int64_t)cols; inner = 1;
        }
    }
    const bool track = requires_grad && GradMode::is_enabled();
    auto result = create(out_shape, track);
    const bool indexed = (op == WM_R_MAX || op == WM_R_MIN);
    std::shared_ptr<int64_t> idx = (indexed && track) ? device_index_buffer((size_t)(outer * inner)) : nullptr;
    ck(wm_reduce(op, data.dev(), outer, n, inner, result->data.dev_write(), idx.get()), "reduction");
    if (track) {
        auto self_ptr = const_cast<Tensor*>(this)->shared_from_this();
        Tensor* res = result.get();
        result->parents = {self_ptr};
        // mean reuses sum's closure: the gradient is not divided by n (:1709-1721).
        const int bop = indexed ? op : WM_R_SUM;
        result->grad_fn = [self_ptr, res, bop, idx, outer, n, inner]() {
            int acc = 0;
            float* gx = grad_target(self_ptr, &acc);
            ck(wm_reduce_bwd(bop, res->grad.dev(), idx.get(), outer, n, inner, gx, acc), "reduction backward");
        };
    }
    return result;
}

TensorPtr Tensor::sum(int dim, bool keepdim) const { return reduce_2d(WM_R_SUM, dim, keepdim, false); }
TensorPtr Tensor::mean(int dim, bool keepdim) const { return reduce_2d(WM_R_MEAN, dim, keepdim, false); }
TensorPtr Tensor::max(int dim, bool keepdim) const { return reduce_2d(WM_R_MAX, dim, keepdim, true); }
TensorPtr Tensor::min(int dim, bool keepdim) const { return reduce_2d(WM_R_MIN, dim, keepdim, true); }

// N-d, negative dims count from the back, fp32 indices, never tracked.
TensorPtr Tensor::arg_reduce(int op, int dim, bool keepdim) const {
    const int nd = (int)shape.size();
    if (dim < 0) dim = nd + dim;
    assert(dim >= 0 && dim < nd);
    std::vector<size_t> out_shape;
    int64_t outer = 1, inner = 1;
    for (int i = 0; i < nd; ++i) {
        if (i == dim) {
            if (keepdim) out_shape.push_back(1);
        } else {
            out_shape.push_back(shape[i]);
        }
        if (i < dim) outer *= (int64_t)shape[i];
        if (i > dim) inner *= (int64_t)shape[i];
    }
    if (out_shape.empty()) out_shape.push_back(1);
    auto result = create(out_shape, false);
    ck(wm_reduce(op, data.dev(), outer, (int64_t)shape[dim], inner, result->data.dev_write(), nullptr), "argmax/argmin");
    return result;
}

TensorPtr Tensor::argmax(int dim, bool keepdim) const { return arg_reduce(WM_R_ARGMAX, dim, keepdim); }
TensorPtr Tensor::argmin(int dim, bool keepdim) const { return arg_reduce(WM_R_ARGMIN, dim, keepdim); }

// ---------------------------------------------------------------------------
// Shape glue: reshape :2250, flatten :2898, squeeze :2916, unsqueeze :2979
// ---------------------------------------------------------------------------

// A copy of the data under a new shape.  copy_grad: the result's gradient
// starts as a copy of this tensor's (reshape's behaviour, :2256-2257).
// The closure adds the result's gradient back element for element.
TensorPtr Tensor::copy_as(const std::vector<size_t>& new_shape, bool result_requires_grad, bool copy_grad) const {
    auto result = create(new_shape, result_requires_grad);
    const int64_t n = (int64_t)data.size();
    if (n) ck(wm_d2d(result->data.dev_write(), data.dev(), (size_t)n * sizeof(float)), "copy");
    if (copy_grad && result_requires_grad) result->grad = grad;
    if (should_track_grad()) {
        auto self_ptr = const_cast<Tensor*>(this)->shared_from_this();
        Tensor* res = result.get();
        result->parents = {self_ptr};
        result->grad_fn = [self_ptr, res, n]() {
            int acc = 0;
            float* gx = grad_target(self_ptr, &acc);
            ck(wm_unary_bwd(WM_SCALE, res->grad.dev(), nullptr, nullptr, gx, acc, n, 1.0f, 0.0f),
               "copy backward");
        };
    }
    return result;
}

TensorPtr Tensor::reshape(const std::vector<size_t>& new_shape) const {
    assert(numel_of(new_shape) == data.size());
    const bool track = requires_grad && GradMode::is_enabled();
    return copy_as(new_shape, track, true);
}

TensorPtr Tensor::flatten(size_t start_dim) const {
    assert(start_dim < shape.size());
    std::vector<size_t> new_shape(shape.begin(), shape.begin() + (std::ptrdiff_t)start_dim);
    size_t flat = 1;
    for (size_t i = start_dim; i < shape.size(); ++i) flat *= shape[i];
    new_shape.push_back(flat);
    return reshape(new_shape);
}

// squeeze/unsqueeze create their result with the input's requires_grad
// (not the grad-mode-aware flag) and only attach a closure when tracking.
TensorPtr Tensor::squeeze(int dim) const {
    std::vector<size_t> new_shape;
    if (dim == -1) {
        for (auto s : shape)
            if (s != 1) new_shape.push_back(s);
        if (new_shape.empty()) new_shape.push_back(1);
    } else {
        const int nd = (int)shape.size();
        if (dim < 0) dim += nd;
        assert(dim >= 0 && dim < nd && "Dimension out of range");
        for (int i = 0; i < nd; ++i)
            if (!(i == dim && shape[i] == 1)) new_shape.push_back(shape[i]);
    }
    return copy_as(new_shape, requires_grad, false);
}

TensorPtr Tensor::unsqueeze(int dim) const {
    const int nd = (int)shape.size();
    if (dim < 0) dim += nd + 1;
    assert(dim >= 0 && dim <= nd && "Dimension out of range");
    std::vector<size_t> new_shape;
    for (int i = 0; i < nd + 1; ++i) {
        if (i == dim) new_shape.push_back(1);
        if (i < nd) new_shape.push_back(shape[i]);
    }
    return copy_as(new_shape, requires_grad, false);
}

// ---------------------------------------------------------------------------
// Matrix products on the matrix cores (include/wm_gemm.h): matmul :783-825,
// bmm :827-895, transpose :2223-2248.  Shape mismatches throw
// std::invalid_argument where the reference asserts.
// ---------------------------------------------------------------------------

TensorPtr Tensor::matmul(const TensorPtr& other) const {
    if (shape.size() != 2 || other->shape.size() != 2) throw std::invalid_argument("matmul: operands must be 2-D");
    if (shape[1] != other->shape[0]) throw std::invalid_argument("matmul: inner dimensions differ");
    const int64_t m = (int64_t)shape[0], k = (int64_t)shape[1], n = (int64_t)other->shape[1];
    const bool track = (requires_grad || other->requires_grad) && GradMode::is_enabled();
    auto result = create({shape[0], other->shape[1]}, track);
    ck(wm_matmul(data.dev(), other->data.dev(), m, k, n, result->data.dev_write()), "matmul");
    if (track) {
        auto self_ptr = const_cast<Tensor*>(this)->shared_from_this();
        auto other_ptr = other;
        Tensor* res = result.get();
        result->parents = {self_ptr, other_ptr};
        result->grad_fn = [self_ptr, other_ptr, res, m, k, n]() {
            // One gradient at a time, so x.matmul(x) adds both into one buffer.
            if (self_ptr->requires_grad) {
                int acc = 0;
                float* ga = grad_target(self_ptr, &acc);
                ck(wm_matmul_bwd(res->grad.dev(), self_ptr->data.dev(), other_ptr->data.dev(), m, k, n, ga, acc,
                                 nullptr, 0),
                   "matmul backward");
            }
            if (other_ptr->requires_grad) {
                int acc = 0;
                float* gb = grad_target(other_ptr, &acc);
                ck(wm_matmul_bwd(res->grad.dev(), self_ptr->data.dev(), other_ptr->data.dev(), m, k, n, nullptr, 0,
                                 gb, acc),
                   "matmul backward");
            }
        };
    }
    return result;
}

TensorPtr Tensor::bmm(const TensorPtr& other) const {
    if (shape.size() != 3 || other->shape.size() != 3) throw std::invalid_argument("bmm requires 3D tensors");
    if (shape[0] != other->shape[0]) throw std::invalid_argument("bmm: batch sizes must match");
    if (shape[2] != other->shape[1]) throw std::invalid_argument("bmm: inner dimensions must match");
    const int64_t batch = (int64_t)shape[0], m = (int64_t)shape[1], k = (int64_t)shape[2],
                  n = (int64_t)other->shape[2];
    const bool track = (requires_grad || other->requires_grad) && GradMode::is_enabled();
    auto result = create({shape[0], shape[1], other->shape[2]}, track);
    ck(wm_bmm(data.dev(), other->data.dev(), batch, m, k, n, result->data.dev_write()), "bmm");
    if (track) {
        auto self_ptr = const_cast<Tensor*>(this)->shared_from_this();
        auto other_ptr = other;
        Tensor* res = result.get();
        result->parents = {self_ptr, other_ptr};
        result->grad_fn = [self_ptr, other_ptr, res, batch, m, k, n]() {
            if (self_ptr->requires_grad) {
                int acc = 0;
                float* ga = grad_target(self_ptr, &acc);
                ck(wm_bmm_bwd(res->grad.dev(), self_ptr->data.dev(), other_ptr->data.dev(), batch, m, k, n, ga, acc,
                              nullptr, 0),
                   "bmm backward");
            }
            if (other_ptr->requires_grad) {
                int acc = 0;
                float* gb = grad_target(other_ptr, &acc);
                ck(wm_bmm_bwd(res->grad.dev(), self_ptr->data.dev(), other_ptr->data.dev(), batch, m, k, n, nullptr,
                              0, gb, acc),
                   "bmm backward");
            }
        };
    }
    return result;
}

TensorPtr Tensor::transpose() const {
    if (shape.size() != 2) throw std::invalid_argument("transpose: tensor must be 2-D");
    const int64_t rows = (int64_t)shape[0], cols = (int64_t)shape[1];
    const bool track = requires_grad && GradMode::is_enabled();
    auto result = create({shape[1], shape[0]}, track);
    ck(wm_transpose2d(data.dev(), rows, cols, result->data.dev_write(), 0), "transpose");
    if (track) {
        auto self_ptr = const_cast<Tensor*>(this)->shared_from_this();
        Tensor* res = result.get();
        result->parents = {self_ptr};
        result->grad_fn = [self_ptr, res, rows, cols]() {
            int acc = 0;
            float* gx = grad_target(self_ptr, &acc);
            ck(wm_transpose2d(res->grad.dev(), cols, rows, gx, acc), "transpose backward");
        };
    }
    return result;
}

// ---------------------------------------------------------------------------
// Outside this build
// ---------------------------------------------------------------------------

TensorPtr Tensor::slice(size_t, size_t, int) const { out_of_scope("slice"); }
TensorPtr Tensor::conv2d(const TensorPtr&, const TensorPtr&, size_t, size_t) const { out_of_scope("conv2d"); }
TensorPtr Tensor::conv_transpose2d(const TensorPtr&, const TensorPtr&, size_t, size_t, size_t) const {
    out_of_scope("conv_transpose2d");
}
TensorPtr Tensor::maxpool2d(size_t, size_t) const { out_of_scope("maxpool2d"); }
TensorPtr Tensor::avgpool2d(size_t, size_t) const { out_of_scope("avgpool2d"); }
TensorPtr Tensor::permute(const std::vector<int>&) const { out_of_scope("permute"); }
TensorPtr Tensor::flip_horizontal() const { out_of_scope("flip_horizontal"); }
TensorPtr Tensor::random_flip_horizontal(float) const { out_of_scope("random_flip_horizontal"); }
TensorPtr Tensor::pad2d(size_t) const { out_of_scope("pad2d"); }
TensorPtr Tensor::crop(size_t, size_t, size_t, size_t) const { out_of_scope("crop"); }
TensorPtr Tensor::random_crop(size_t, size_t) const { out_of_scope("random_crop"); }

// print (:2294-2310): shape, and the values of tensors of at most 10 elements.
void Tensor::print(const char* name) const {
    if (name) printf("%s: ", name);
    printf("Tensor(shape=[");
    for (size_t i = 0; i < shape.size(); i++) printf("%zu%s", shape[i], i < shape.size() - 1 ? ", " : "");
    printf("]");
    if (data.size() <= 10) {
        printf(", data=[");
        for (size_t i = 0; i < data.size(); i++) printf("%.4f%s", data[i], i < data.size() - 1 ? ", " : "");
        printf("]");
    }
    printf(")\n");
}

TensorPtr operator*(float scalar, const TensorPtr& t) { return t->mul(scalar); }
