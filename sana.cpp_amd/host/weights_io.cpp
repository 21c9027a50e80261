// GGUF weight index and payload reads of the drop-in API, on this library's
// own GGUF reader (csrc/gguf.h).  Conventions kept from the reference
// (src/weights_io.cpp:121-164, :325-377): shapes reported in PyTorch order,
// absolute payload offsets, linear weights transposed to [in, out].
#include "weights_io.h"

#include <cstring>
#include <fstream>
#include <stdexcept>

#include "../csrc/gguf.h"

namespace {

const char * dtype_name(uint32_t ggml_type) {
    switch (ggml_type) {
        case sana::gguf::kF32: return "float32";
        case sana::gguf::kF16: return "float16";
        case sana::gguf::kBF16: return "bfloat16";
        default: return nullptr;
    }
}

float half_to_float(uint16_t h) {
    const uint32_t sign = (uint32_t)(h & 0x8000u) << 16;
    uint32_t exp = (h >> 10) & 0x1fu, man = h & 0x3ffu;
    uint32_t bits;
    if (exp == 0) {
        if (man == 0) {
            bits = sign;
        } else {  // subnormal: renormalise
            exp = 127 - 15 + 1;
            while ((man & 0x400u) == 0) {
                man <<= 1;
                --exp;
            }
            man &= 0x3ffu;
            bits = sign | (exp << 23) | (man << 13);
        }
    } else if (exp == 31) {
        bits = sign | 0x7f800000u | (man << 13);
    } else {
        bits = sign | ((exp + 127 - 15) << 23) | (man << 13);
    }
    float f;
    std::memcpy(&f, &bits, 4);
    return f;
}

}  // namespace

bool ends_with(const std::string & value, const std::string & suffix) {
    return value.size() >= suffix.size() && value.compare(value.size() - suffix.size(), suffix.size(), suffix) == 0;
}

std::unordered_map<std::string, SavedWeightInfo> load_weight_index(const std::string & path) {
    if (!ends_with(path, ".gguf"))
        throw std::runtime_error("only .gguf weight files are supported by this build: " + path);
    const sana::gguf::Index idx = sana::gguf::read_index(path);
    std::unordered_map<std::string, SavedWeightInfo> out;
    for (const auto & t : idx.tensors) {
        SavedWeightInfo info;
        info.file = path;
        for (int64_t d : t.shape) info.shape.push_back(static_cast<size_t>(d));
        const char * dt = dtype_name(t.type);
        info.dtype = dt ? dt : "ggml_type_" + std::to_string(t.type);
        info.format = WeightFormat::Gguf;
        info.offset = static_cast<size_t>(t.offset);
        out[t.name] = info;
    }
    return out;
}

Tensor load_weight_tensor(const std::string & /*weights_dir*/,
                          const std::unordered_map<std::string, SavedWeightInfo> & index, const std::string & name) {
    auto it = index.find(name);
    if (it == index.end()) throw std::invalid_argument("weight name not found in weight index");
    const SavedWeightInfo & info = it->second;
    if (info.format != WeightFormat::Gguf) throw std::runtime_error("only gguf weights are supported by this build");
    const size_t esize = info.dtype == "float32" ? 4 : (info.dtype == "float16" || info.dtype == "bfloat16") ? 2 : 0;
    if (esize == 0) throw std::runtime_error("unsupported gguf tensor type " + info.dtype + " for: " + name);
    Tensor t(info.shape);
    std::ifstream in(info.file, std::ios::binary);
    if (!in) throw std::runtime_error("failed to open gguf weight file: " + info.file);
    in.seekg(static_cast<std::streamoff>(info.offset));
    std::vector<float> & dst = t.data();
    if (esize == 4) {
        in.read(reinterpret_cast<char *>(dst.data()), static_cast<std::streamsize>(dst.size() * 4));
    } else {
        std::vector<uint16_t> raw(dst.size());
        in.read(reinterpret_cast<char *>(raw.data()), static_cast<std::streamsize>(raw.size() * 2));
        for (size_t i = 0; i < raw.size(); ++i) {
            if (info.dtype == "float16") {
                dst[i] = half_to_float(raw[i]);
            } else {
                const uint32_t bits = (uint32_t)raw[i] << 16;
                std::memcpy(&dst[i], &bits, 4);
            }
        }
    }
    if (!in) throw std::runtime_error("failed to read gguf tensor payload for: " + name);
    return t;
}

Tensor load_linear_weight_tensor(const std::string & weights_dir,
                                 const std::unordered_map<std::string, SavedWeightInfo> & index,
                                 const std::string & name) {
    Tensor w = load_weight_tensor(weights_dir, index, name);
    if (w.rank() != 2) throw std::invalid_argument("linear weight must be rank 2");
    return w.transpose_2d();
}
