// serialize.h -- drop-in for whitematter's core/serialize.h on MI355X.
//
// Same declarations, magic numbers and include guard as the reference
// header (core/serialize.h:1-46), and byte-identical files: the WMT tensor,
// WMM model, WMO optimizer and checkpoint formats are unchanged.  What
// differs is where the floats go: every payload streams between the file
// and device memory through include/wm_io.h (pinned double buffering, no
// host copy of the tensor), so load_tensor / load_model / load_optimizer /
// load_checkpoint fill HBM directly and the save functions read it there.
#ifndef SERIALIZE_H
#define SERIALIZE_H

#include <cstdint>
#include <fstream>
#include <string>

#include "layer.h"
#include "optimizer.h"
#include "tensor.h"

// File format magic numbers for validation
constexpr uint32_t TENSOR_MAGIC = 0x574D5400;  // "WMT\0"
constexpr uint32_t MODEL_MAGIC = 0x574D4D00;   // "WMM\0"
constexpr uint32_t OPTIM_MAGIC = 0x574D4F00;   // "WMO\0"

// Tensor serialization
bool save_tensor(const TensorPtr& tensor, const std::string& path);
bool save_tensor(const TensorPtr& tensor, std::ofstream& out);
TensorPtr load_tensor(const std::string& path);
TensorPtr load_tensor(std::ifstream& in);

// Model serialization (all parameters, in parameters() order)
bool save_model(Module* module, const std::string& path);
bool load_model(Module* module, const std::string& path);

// Optimizer state serialization (SGD and Adam, as the reference)
bool save_optimizer(Optimizer* optimizer, const std::string& path);
bool load_optimizer(Optimizer* optimizer, const std::string& path);

// Checkpoint: model + optimizer state together
struct Checkpoint {
    int epoch;
    float loss;
    float accuracy;
};

bool save_checkpoint(const std::string& path, Module* model, Optimizer* optimizer, int epoch, float loss = 0.0f,
                     float accuracy = 0.0f);
bool load_checkpoint(const std::string& path, Module* model, Optimizer* optimizer, Checkpoint& info);

#endif  // SERIALIZE_H
