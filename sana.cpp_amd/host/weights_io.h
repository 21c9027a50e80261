// Weight index and tensor loading of the drop-in C++ API: the GGUF part of the
// reference's src/weights_io.h:9-42 (same types and function signatures).
// The index comes from this library's own GGUF v2/v3 reader (no ggml).  The
// reference's legacy npy + JSON index and its npy/golden-compare debugging
// helpers are not part of the DiT path and are not provided.
#pragma once

#include <string>
#include <unordered_map>
#include <vector>

#include "tensor.h"

struct TensorComparison {
    float max_abs_diff;
    float mean_abs_diff;
};

enum class WeightFormat {
    Npy,
    Gguf,
};

struct SavedWeightInfo {
    std::string file;           // the .gguf file path
    std::vector<size_t> shape;  // PyTorch order (GGUF ne reversed)
    std::string dtype;          // "float32", "float16" or "bfloat16"
    WeightFormat format = WeightFormat::Npy;
    size_t offset = 0;          // absolute byte offset of the tensor payload in `file`
};

bool ends_with(const std::string & value, const std::string & suffix);

// GGUF files only (".gguf"); anything else throws std::runtime_error.
std::unordered_map<std::string, SavedWeightInfo> load_weight_index(const std::string & path);
// Reads one tensor as fp32.  F32 payloads are read as is; F16 and BF16
// payloads are widened to fp32 (the reference reads every payload as F32).
Tensor load_weight_tensor(const std::string & weights_dir,
                          const std::unordered_map<std::string, SavedWeightInfo> & index, const std::string & name);
// A linear weight ([out, in] in the file) transposed to [in, out].
Tensor load_linear_weight_tensor(const std::string & weights_dir,
                                 const std::unordered_map<std::string, SavedWeightInfo> & index,
                                 const std::string & name);
