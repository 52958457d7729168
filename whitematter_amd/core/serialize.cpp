// serialize.cpp -- WMT / WMM / WMO / checkpoint files for the drop-in
// serialize.h (reference core/serialize.cpp:1-507 defines the formats).
//
// Every format is described once, as an ordered list of fields, by a
// function that takes a `Wire`: a Wire bound to an output file writes each
// field from the object, one bound to an input file reads each field into
// it.  save_* and load_* run the same description, so a field cannot be
// added, dropped or reordered in one direction only.  What differs between
// loaders -- which counts and sizes a file must match, whether a wrong
// optimizer kind refuses the file or is skipped with a warning -- is data in
// the `StateChecks` tables below, not code paths.
//
// Layout (little-endian 4-byte words; float payloads are raw fp32):
//   tensor record  ndim:u32, dims:u32[ndim], values:f32[prod(dims)]
//   WMT            TENSOR_MAGIC, tensor record
//   WMM            MODEL_MAGIC, count:u32, tensor record[count]
//   state list     count:u32 (absent for Adam's v list, which reuses m's),
//                  then per buffer size:u32, values:f32[size]
//   SGD state      kind 1:u32, lr:f32, momentum:f32, velocity state list
//   Adam state     kind 2:u32, lr, beta1, beta2, eps:f32, t:i32, m list, v list
//   WMO            OPTIM_MAGIC, SGD or Adam state
//   checkpoint     MODEL_MAGIC, version 1:u32, epoch:i32, loss:f32,
//                  accuracy:f32, count:u32, tensor record[count],
//                  has_state:u32, [SGD or Adam state]
//
// Float payloads never pass through a host vector: they stream between the
// fstream and the DeviceVector's device memory through wm_read_into_device /
// wm_write_from_device (pinned double buffering on the library stream).  A
// payload transfer is not checked on its own: a short read or a refused
// write leaves the stream failed, and the next field (or the final stream
// check) reports it, which is where the reference's functions fail too.
#include "serialize.h"

#include <cstdio>
#include <stdexcept>
#include <string>

#include "wm_hip.h"
#include "wm_io.h"

namespace {

// ---------------------------------------------------------------------------
// A field codec over one open file, in one direction.
// ---------------------------------------------------------------------------

int64_t pull_from_istream(void* ctx, void* buf, int64_t n) {
    auto* in = static_cast<std::ifstream*>(ctx);
    in->read(static_cast<char*>(buf), (std::streamsize)n);
    return (int64_t)in->gcount();
}

int64_t push_to_ostream(void* ctx, const void* buf, int64_t n) {
    auto* out = static_cast<std::ofstream*>(ctx);
    out->write(static_cast<const char*>(buf), (std::streamsize)n);
    return out->good() ? n : 0;
}

class Wire {
public:
    explicit Wire(std::ofstream& f) : out_(&f) {}
    explicit Wire(std::ifstream& f) : in_(&f) {}

    bool reading() const { return in_ != nullptr; }
    bool good() const { return reading() ? in_->good() : out_->good(); }
    std::ifstream& in() { return *in_; }
    std::ofstream& out() { return *out_; }

    // One 4-byte word (uint32_t, int or float): written from v, or read into
    // v.  False when the stream has failed afterwards.
    template <class T>
    bool word(T& v) {
        static_assert(sizeof(T) == 4, "fields are 4-byte words");
        if (reading()) in_->read(reinterpret_cast<char*>(&v), sizeof v);
        else out_->write(reinterpret_cast<const char*>(&v), sizeof v);
        return good();
    }
    // A word the writer derives from the object (a count, a size, a tag)
    // and the reader only learns from the file.
    bool derived(uint32_t from_object, uint32_t& from_file) {
        from_file = from_object;
        return word(from_file);
    }

    // The values of v, straight between the file and device memory.
    void payload(wm::DeviceVector& v) {
        const int64_t bytes = (int64_t)(v.size() * sizeof(float));
        const int rc = reading() ? wm_read_into_device(pull_from_istream, in_, v.dev_write(), bytes)
                                 : wm_write_from_device(push_to_ostream, out_, v.dev(), bytes);
        // WM_ERR_IO is the short file / refusing stream case, carried by
        // the stream state; anything else is a device failure.
        if (rc != WM_OK && rc != WM_ERR_IO)
            throw std::runtime_error(std::string("whitematter_amd ") + (reading() ? "load" : "save") + ": " +
                                     wm_last_error());
    }

private:
    std::ofstream* out_ = nullptr;
    std::ifstream* in_ = nullptr;
};

// ---------------------------------------------------------------------------
// Loader rules: which file fields must agree with the object, and what a
// mismatch prints.  A null message means the field is taken as it comes.
// ---------------------------------------------------------------------------

struct ListChecks {
    const char* count_mismatch;  // count in the file != number of buffers
    const char* size_mismatch;   // size in the file != the buffer's size
};

struct StateChecks {
    bool refuse_other_kind;      // a file of the other optimizer kind: refuse (true) or skip (false)
    const char* other_kind_fmt;  // printed for it; both %s are the file's kind name
    ListChecks sgd_velocity, adam_m, adam_v;
};

// WMO files are checked buffer for buffer (core/serialize.cpp:239-316).
const StateChecks kOptimizerFile = {
    true, "Error: File contains %s state but optimizer is not %s\n",
    {"Error: Velocity buffer count mismatch\n", "Error: Velocity buffer size mismatch\n"},
    {"Error: Adam buffer count mismatch\n", "Error: Adam m buffer size mismatch\n"},
    {nullptr, "Error: Adam v buffer size mismatch\n"},
};

// Checkpoints take the state as it comes: counts and sizes are read and not
// compared, each buffer reads its own size's worth of floats, and state of
// the other kind is skipped (core/serialize.cpp:459-500).
const StateChecks kCheckpoint = {
    false, "Warning: Checkpoint has %s state but optimizer is not %s, skipping\n",
    {nullptr, nullptr}, {nullptr, nullptr}, {nullptr, nullptr},
};

bool refuse(const char* msg) {
    fputs(msg, stderr);
    return false;
}

// ---------------------------------------------------------------------------
// Format descriptions, one per record kind, shared by both directions.
// ---------------------------------------------------------------------------

// A list of optimizer state buffers.  `counted` is false for Adam's v list,
// whose count is m's.
bool state_list(Wire& w, std::vector<wm::DeviceVector>& bufs, bool counted, const ListChecks& chk) {
    if (counted) {
        uint32_t n;
        if (!w.derived((uint32_t)bufs.size(), n)) return false;
        if (w.reading() && chk.count_mismatch && n != bufs.size()) return refuse(chk.count_mismatch);
    }
    for (auto& b : bufs) {
        uint32_t n;
        if (!w.derived((uint32_t)b.size(), n)) return false;
        if (w.reading() && chk.size_mismatch && n != b.size()) return refuse(chk.size_mismatch);
        w.payload(b);
    }
    return true;
}

bool sgd_fields(Wire& w, SGD& s, const StateChecks& chk) {
    return w.word(s.lr) && w.word(s.momentum) && state_list(w, s.velocity, true, chk.sgd_velocity);
}

bool adam_fields(Wire& w, Adam& a, const StateChecks& chk) {
    return w.word(a.lr) && w.word(a.beta1) && w.word(a.beta2) && w.word(a.eps) && w.word(a.t) &&
           state_list(w, a.m, true, chk.adam_m) && state_list(w, a.v, false, chk.adam_v);
}

// The optimizer kinds a file can hold, by their tag in the file.
struct StateKind {
    uint32_t tag;
    const char* name;
    bool (*fields)(Wire&, Optimizer*, const StateChecks&);
    bool (*holds)(Optimizer*);
};

const StateKind kKinds[] = {
    {1, "SGD", [](Wire& w, Optimizer* o, const StateChecks& c) { return sgd_fields(w, *static_cast<SGD*>(o), c); },
     [](Optimizer* o) { return dynamic_cast<SGD*>(o) != nullptr; }},
    {2, "Adam", [](Wire& w, Optimizer* o, const StateChecks& c) { return adam_fields(w, *static_cast<Adam*>(o), c); },
     [](Optimizer* o) { return dynamic_cast<Adam*>(o) != nullptr; }},
};

const StateKind* kind_of(Optimizer* o) {
    for (const auto& k : kKinds)
        if (k.holds(o)) return &k;
    return nullptr;
}

const StateKind* kind_tagged(uint32_t tag) {
    for (const auto& k : kKinds)
        if (k.tag == tag) return &k;
    return nullptr;
}

enum class State { done, failed, unknown_kind };

// An optimizer state block: its kind tag, then that kind's fields.  Writing
// needs an optimizer of a known kind (unknown_kind otherwise, nothing
// written).  Reading an unknown tag gives unknown_kind; a known tag the
// optimizer is not follows chk (refuse, or skip the block's fields).  `tag`
// is the block's tag as written or read.
State state_block(Wire& w, Optimizer* opt, const StateChecks& chk, uint32_t& tag) {
    const StateKind* mine = kind_of(opt);
    if (!w.reading() && !mine) return State::unknown_kind;
    if (!w.derived(mine ? mine->tag : 0u, tag)) return State::failed;
    const StateKind* filed = kind_tagged(tag);
    if (!filed) return State::unknown_kind;
    if (filed != mine) {
        fprintf(stderr, chk.other_kind_fmt, filed->name, filed->name);
        return chk.refuse_other_kind ? State::failed : State::done;
    }
    return filed->fields(w, opt, chk) ? State::done : State::failed;
}

// A tensor record.  Reading creates the tensor (shape from the file,
// requires_grad, values straight into its device storage).
bool tensor_record(Wire& w, TensorPtr& t) {
    uint32_t ndim;
    if (!w.derived(w.reading() ? 0u : (uint32_t)t->shape.size(), ndim)) return false;
    std::vector<size_t> shape(w.reading() ? ndim : 0);
    for (uint32_t d = 0; d < ndim; ++d) {
        uint32_t extent;
        if (!w.derived(w.reading() ? 0u : (uint32_t)t->shape[d], extent)) return false;
        if (w.reading()) shape[d] = extent;
    }
    if (w.reading()) t = Tensor::create(shape, true);
    w.payload(t->data);
    return w.good();
}

// A module's parameters, in parameters() order.  Reading requires the
// file's count and every record's shape to match the module, then moves
// each record's storage into the parameter.
bool parameter_list(Wire& w, Module* module) {
    auto params = module->parameters();
    uint32_t n;
    if (!w.derived((uint32_t)params.size(), n)) return false;
    if (w.reading() && n != params.size()) {
        fprintf(stderr, "Error: Parameter count mismatch. File has %u, model has %zu\n", n, params.size());
        return false;
    }
    for (size_t i = 0; i < n; ++i) {
        if (!w.reading()) {
            if (!save_tensor(params[i], w.out())) return false;
            continue;
        }
        TensorPtr rec = load_tensor(w.in());
        if (!rec) return false;
        if (rec->shape != params[i]->shape) {
            fprintf(stderr, "Error: Shape mismatch for parameter %zu\n", i);
            return false;
        }
        params[i]->data = std::move(rec->data);
    }
    return true;
}

// ---------------------------------------------------------------------------
// Files: open, then the leading magic word (written, or read and checked).
// ---------------------------------------------------------------------------

bool open_for_write(std::ofstream& f, const std::string& path) {
    f.open(path, std::ios::binary);
    if (f.is_open()) return true;
    fprintf(stderr, "Error: Cannot open file for writing: %s\n", path.c_str());
    return false;
}

bool open_for_read(std::ifstream& f, const std::string& path) {
    f.open(path, std::ios::binary);
    if (f.is_open()) return true;
    fprintf(stderr, "Error: Cannot open file for reading: %s\n", path.c_str());
    return false;
}

// `what` names the file kind in the refusal ("tensor", "model", ...).
bool magic(Wire& w, uint32_t expected, const char* what, const std::string& path) {
    uint32_t m = expected;
    if (w.word(m) && m == expected) return true;
    if (w.reading()) fprintf(stderr, "Error: Invalid %s file format: %s\n", what, path.c_str());
    return false;
}

// The checkpoint header after its magic: version, epoch, loss, accuracy.
bool checkpoint_header(Wire& w, Checkpoint& info) {
    uint32_t version = 1;
    if (!w.word(version) || version != 1) {
        if (w.reading()) fprintf(stderr, "Error: Unsupported checkpoint version: %u\n", version);
        return false;
    }
    return w.word(info.epoch) && w.word(info.loss) && w.word(info.accuracy);
}

// The checkpoint's optional state: a has-state word, then the block.  An
// optimizer of a kind no tag names is written as has-state 1 with no block
// (the reference writes the same), and a block whose tag no kind knows is
// ignored when reading.
bool checkpoint_state(Wire& w, Optimizer* opt) {
    uint32_t has;
    if (!w.derived(opt ? 1u : 0u, has)) return false;
    if (!has || !opt) return true;
    uint32_t tag;
    return state_block(w, opt, kCheckpoint, tag) != State::failed;
}

}  // namespace

// ---- tensors (core/serialize.cpp:36-108) --------------------------------------

bool save_tensor(const TensorPtr& tensor, std::ofstream& out) {
    if (!tensor || !out.good()) return false;
    Wire w(out);
    TensorPtr t = tensor;
    return tensor_record(w, t);
}

bool save_tensor(const TensorPtr& tensor, const std::string& path) {
    std::ofstream f;
    if (!open_for_write(f, path)) return false;
    Wire w(f);
    return magic(w, TENSOR_MAGIC, "tensor", path) && save_tensor(tensor, f);
}

TensorPtr load_tensor(std::ifstream& in) {
    if (!in.good()) return nullptr;
    Wire w(in);
    TensorPtr t;
    return tensor_record(w, t) ? t : nullptr;
}

TensorPtr load_tensor(const std::string& path) {
    std::ifstream f;
    if (!open_for_read(f, path)) return nullptr;
    Wire w(f);
    return magic(w, TENSOR_MAGIC, "tensor", path) ? load_tensor(f) : nullptr;
}

// ---- models (:111-181) ----------------------------------------------------------

bool save_model(Module* module, const std::string& path) {
    if (!module) return false;
    std::ofstream f;
    if (!open_for_write(f, path)) return false;
    Wire w(f);
    if (!magic(w, MODEL_MAGIC, "model", path) || !parameter_list(w, module)) return false;
    printf("Model saved: %zu parameters to %s\n", module->parameters().size(), path.c_str());
    return true;
}

bool load_model(Module* module, const std::string& path) {
    if (!module) return false;
    std::ifstream f;
    if (!open_for_read(f, path)) return false;
    Wire w(f);
    if (!magic(w, MODEL_MAGIC, "model", path) || !parameter_list(w, module)) return false;
    printf("Model loaded: %zu parameters from %s\n", module->parameters().size(), path.c_str());
    return true;
}

// ---- optimizer state (:184-316) -------------------------------------------------

bool save_optimizer(Optimizer* optimizer, const std::string& path) {
    if (!optimizer) return false;
    std::ofstream f;
    if (!open_for_write(f, path)) return false;
    Wire w(f);
    if (!magic(w, OPTIM_MAGIC, "optimizer", path)) return false;
    uint32_t tag;
    switch (state_block(w, optimizer, kOptimizerFile, tag)) {
        case State::failed: return false;
        case State::unknown_kind: return refuse("Error: Unknown optimizer type\n");
        case State::done: break;
    }
    printf("Optimizer state saved to %s\n", path.c_str());
    return w.good();
}

bool load_optimizer(Optimizer* optimizer, const std::string& path) {
    if (!optimizer) return false;
    std::ifstream f;
    if (!open_for_read(f, path)) return false;
    Wire w(f);
    if (!magic(w, OPTIM_MAGIC, "optimizer", path)) return false;
    uint32_t tag;
    switch (state_block(w, optimizer, kOptimizerFile, tag)) {
        case State::failed: return false;
        case State::unknown_kind:
            fprintf(stderr, "Error: Unknown optimizer type in file: %u\n", tag);
            return false;
        case State::done: break;
    }
    printf("Optimizer state loaded from %s\n", path.c_str());
    return w.good();
}

// ---- checkpoints (:319-507) ------------------------------------------------------

bool save_checkpoint(const std::string& path, Module* model, Optimizer* optimizer, int epoch, float loss,
                     float accuracy) {
    std::ofstream f;
    if (!open_for_write(f, path)) return false;
    Wire w(f);
    Checkpoint info{epoch, loss, accuracy};
    if (!magic(w, MODEL_MAGIC, "checkpoint", path) || !checkpoint_header(w, info) || !parameter_list(w, model) ||
        !checkpoint_state(w, optimizer))
        return false;
    printf("Checkpoint saved: epoch=%d, loss=%.4f, accuracy=%.2f%% to %s\n", epoch, loss, accuracy * 100.0f,
           path.c_str());
    return w.good();
}

bool load_checkpoint(const std::string& path, Module* model, Optimizer* optimizer, Checkpoint& info) {
    std::ifstream f;
    if (!open_for_read(f, path)) return false;
    Wire w(f);
    if (!magic(w, MODEL_MAGIC, "checkpoint", path) || !checkpoint_header(w, info) || !parameter_list(w, model) ||
        !checkpoint_state(w, optimizer))
        return false;
    printf("Checkpoint loaded: epoch=%d, loss=%.4f, accuracy=%.2f%% from %s\n", info.epoch, info.loss,
           info.accuracy * 100.0f, path.c_str());
    return w.good();
}
