// GGUF (v2/v3) tensor index reader, written from the published GGUF layout:
//   "GGUF" magic, u32 version, u64 tensor count, u64 metadata count,
//   metadata key/value pairs (typed, arrays nested), tensor infos
//   (name, u32 n_dims, u64 ne[n_dims] fastest axis first, u32 ggml type,
//   u64 offset relative to the data section), then the data section starting
//   at the next multiple of general.alignment (default 32).
// This replaces the ggml gguf_* calls of load_gguf_weight_index
// (src/weights_io.cpp:134-164): shapes are reported in PyTorch order (ne
// reversed, :125-132) and offsets as absolute file offsets (data offset +
// tensor offset, :157).
#pragma once

#include <cstdint>
#include <map>
#include <string>
#include <vector>

namespace sana {
namespace gguf {

enum GgmlType : uint32_t { kF32 = 0, kF16 = 1, kBF16 = 30 };

struct TensorInfo {
    std::string name;
    std::vector<int64_t> shape;  // PyTorch order
    uint32_t type = 0;
    uint64_t offset = 0;         // absolute byte offset in the file
    uint64_t nbytes = 0;         // payload size (F32/F16/BF16), 0 for other types
};

// One metadata value: a scalar (number in `num`, text in `str`) or an array
// of scalars (`nums` / `strs`, element type in `elem_type`).
struct MetaValue {
    uint32_t type = 0;       // GGUF value type; 9 = array
    uint32_t elem_type = 0;  // arrays
    double num = 0.0;
    std::string str;
    std::vector<double> nums;
    std::vector<std::string> strs;
};

struct Index {
    std::string path;
    std::map<std::string, MetaValue> meta;  // every key except arrays of arrays
    uint32_t version = 0;
    uint64_t alignment = 32;
    uint64_t data_offset = 0;
    uint64_t file_size = 0;
    std::vector<TensorInfo> tensors;
};

// Throws std::runtime_error with a message naming the file on any malformed
// or truncated input.
Index read_index(const std::string & path);

// Read-only memory map of a whole file.
class MappedFile {
public:
    explicit MappedFile(const std::string & path);
    ~MappedFile();
    MappedFile(const MappedFile &) = delete;
    MappedFile & operator=(const MappedFile &) = delete;
    const unsigned char * data() const { return data_; }
    uint64_t size() const { return size_; }

private:
    const unsigned char * data_ = nullptr;
    uint64_t size_ = 0;
};

// The payload of tensor t as fp32: F32 is returned in place (pointer into the
// mapping); F16 and BF16 are widened into `tmp` (exactly: both are subsets of
// fp32).  Throws std::runtime_error naming the tensor for any other type.
const float * payload_f32(const MappedFile & f, const TensorInfo & t, std::vector<float> & tmp);

// Block prefixes as find_block_prefixes (src/transformer.cpp:401-426): the
// names ending in ".scale_shift_table", minus that suffix, ordered by trailing
// integer when two prefixes share a stem, else lexicographically.
std::vector<std::string> block_prefixes(const std::vector<std::string> & names);

}  // namespace gguf
}  // namespace sana
