// GGUF index reader and mmap helper; see gguf.h for the format summary.
#include "gguf.h"

#include <fcntl.h>
#include <sys/mman.h>
#include <sys/stat.h>
#include <unistd.h>

#include <algorithm>
#include <cstring>
#include <set>
#include <stdexcept>

namespace sana {
namespace gguf {
namespace {

enum ValueType : uint32_t {
    kU8 = 0, kI8 = 1, kU16 = 2, kI16 = 3, kU32 = 4, kI32 = 5, kF32v = 6, kBool = 7, kString = 8, kArray = 9,
    kU64 = 10, kI64 = 11, kF64 = 12,
};

struct Reader {
    const unsigned char * p;
    uint64_t n, pos = 0;
    const std::string & path;

    void need(uint64_t k) {
        if (k > n || pos > n - k) throw std::runtime_error("truncated gguf file: " + path);
    }
    template <class T>
    T get() {
        need(sizeof(T));
        T v;
        std::memcpy(&v, p + pos, sizeof(T));
        pos += sizeof(T);
        return v;
    }
    std::string str() {
        const uint64_t len = get<uint64_t>();
        need(len);
        std::string s(reinterpret_cast<const char *>(p + pos), len);
        pos += len;
        return s;
    }
    double number(uint32_t t) {
        switch (t) {
            case kU8: return get<uint8_t>();
            case kI8: return get<int8_t>();
            case kBool: return get<uint8_t>() ? 1.0 : 0.0;
            case kU16: return get<uint16_t>();
            case kI16: return get<int16_t>();
            case kU32: return get<uint32_t>();
            case kI32: return get<int32_t>();
            case kF32v: return get<float>();
            case kU64: return (double)get<uint64_t>();
            case kI64: return (double)get<int64_t>();
            case kF64: return get<double>();
            default: throw std::runtime_error("not a numeric gguf metadata type in " + path);
        }
    }
    // Reads one value into v (arrays of scalars and strings; nested arrays skipped).
    void value(uint32_t t, MetaValue & v) {
        v.type = t;
        if (t == kString) {
            v.str = str();
        } else if (t == kArray) {
            const uint32_t et = get<uint32_t>();
            const uint64_t cnt = get<uint64_t>();
            v.elem_type = et;
            if (et == kArray) {
                for (uint64_t i = 0; i < cnt; ++i) skip_value(et, 1);
            } else if (et == kString) {
                if (cnt > n) throw std::runtime_error("implausible gguf array length in " + path);
                v.strs.reserve(cnt);
                for (uint64_t i = 0; i < cnt; ++i) v.strs.push_back(str());
            } else {
                if (cnt > n) throw std::runtime_error("implausible gguf array length in " + path);
                v.nums.reserve(cnt);
                for (uint64_t i = 0; i < cnt; ++i) v.nums.push_back(number(et));
            }
        } else {
            v.num = number(t);
        }
    }
    void skip_value(uint32_t t, int depth = 0) {
        switch (t) {
            case kU8: case kI8: case kBool: need(1); pos += 1; break;
            case kU16: case kI16: need(2); pos += 2; break;
            case kU32: case kI32: case kF32v: need(4); pos += 4; break;
            case kU64: case kI64: case kF64: need(8); pos += 8; break;
            case kString: (void)str(); break;
            case kArray: {
                if (depth > 4) throw std::runtime_error("gguf array nesting too deep: " + path);
                const uint32_t et = get<uint32_t>();
                const uint64_t cnt = get<uint64_t>();
                for (uint64_t i = 0; i < cnt; ++i) skip_value(et, depth + 1);
                break;
            }
            default: throw std::runtime_error("unknown gguf metadata type in " + path);
        }
    }
};

}  // namespace

MappedFile::MappedFile(const std::string & path) {
    const int fd = ::open(path.c_str(), O_RDONLY);
    if (fd < 0) throw std::runtime_error("failed to open gguf weight file: " + path);
    struct stat st;
    if (::fstat(fd, &st) != 0) {
        ::close(fd);
        throw std::runtime_error("failed to stat gguf weight file: " + path);
    }
    size_ = static_cast<uint64_t>(st.st_size);
    if (size_ > 0) {
        void * m = ::mmap(nullptr, size_, PROT_READ, MAP_PRIVATE, fd, 0);
        if (m == MAP_FAILED) {
            ::close(fd);
            throw std::runtime_error("failed to map gguf weight file: " + path);
        }
        data_ = static_cast<const unsigned char *>(m);
    }
    ::close(fd);
}

MappedFile::~MappedFile() {
    if (data_) ::munmap(const_cast<unsigned char *>(data_), size_);
}

Index read_index(const std::string & path) {
    MappedFile f(path);
    Reader r{f.data(), f.size(), 0, path};
    Index idx;
    idx.path = path;
    idx.file_size = f.size();
    if (r.get<uint32_t>() != 0x46554747u) throw std::runtime_error("not a gguf file (bad magic): " + path);
    idx.version = r.get<uint32_t>();
    if (idx.version != 2 && idx.version != 3) throw std::runtime_error("unsupported gguf version in " + path);
    const uint64_t n_tensors = r.get<uint64_t>();
    const uint64_t n_kv = r.get<uint64_t>();
    if (n_tensors > (1u << 24) || n_kv > (1u << 24)) throw std::runtime_error("implausible gguf counts: " + path);
    for (uint64_t i = 0; i < n_kv; ++i) {
        const std::string key = r.str();
        const uint32_t t = r.get<uint32_t>();
        if (key == "general.alignment") {
            if (t != kU32) throw std::runtime_error("general.alignment must be u32: " + path);
            idx.alignment = r.get<uint32_t>();
            if (idx.alignment == 0 || (idx.alignment & (idx.alignment - 1)))
                throw std::runtime_error("general.alignment must be a power of two: " + path);
        } else {
            r.value(t, idx.meta[key]);
        }
    }
    std::set<std::string> seen;
    for (uint64_t i = 0; i < n_tensors; ++i) {
        TensorInfo ti;
        ti.name = r.str();
        const uint32_t nd = r.get<uint32_t>();
        if (nd == 0 || nd > 4) throw std::runtime_error("bad tensor rank for " + ti.name + " in " + path);
        std::vector<int64_t> ne(nd);
        for (uint32_t d = 0; d < nd; ++d) {
            const uint64_t v = r.get<uint64_t>();
            if (v == 0 || v > (1ull << 40)) throw std::runtime_error("bad tensor dim for " + ti.name);
            ne[d] = static_cast<int64_t>(v);
        }
        ti.shape.assign(ne.rbegin(), ne.rend());
        ti.type = r.get<uint32_t>();
        ti.offset = r.get<uint64_t>();
        if (!seen.insert(ti.name).second) throw std::runtime_error("duplicate tensor " + ti.name + " in " + path);
        uint64_t numel = 1;
        for (int64_t v : ti.shape) numel *= static_cast<uint64_t>(v);
        ti.nbytes = ti.type == kF32 ? numel * 4 : (ti.type == kF16 || ti.type == kBF16) ? numel * 2 : 0;
        idx.tensors.push_back(ti);
    }
    idx.data_offset = (r.pos + idx.alignment - 1) / idx.alignment * idx.alignment;
    for (TensorInfo & ti : idx.tensors) {
        if (ti.offset % idx.alignment) throw std::runtime_error("misaligned tensor data for " + ti.name);
        ti.offset += idx.data_offset;
        if (ti.nbytes && (ti.offset > idx.file_size || ti.nbytes > idx.file_size - ti.offset))
            throw std::runtime_error("failed to read gguf tensor payload for: " + ti.name);
    }
    return idx;
}

namespace {
bool trailing_index(const std::string & p, std::string * stem, uint64_t * idx) {
    const size_t dot = p.rfind('.');
    if (dot == std::string::npos || dot + 1 >= p.size()) return false;
    for (size_t i = dot + 1; i < p.size(); ++i)
        if (p[i] < '0' || p[i] > '9') return false;
    *stem = p.substr(0, dot);
    *idx = std::stoull(p.substr(dot + 1));
    return true;
}
}  // namespace

std::vector<std::string> block_prefixes(const std::vector<std::string> & names) {
    const std::string suf = ".scale_shift_table";
    std::set<std::string> u;
    for (const std::string & n : names)
        if (n.size() >= suf.size() && n.compare(n.size() - suf.size(), suf.size(), suf) == 0)
            u.insert(n.substr(0, n.size() - suf.size()));
    std::vector<std::string> v(u.begin(), u.end());
    std::sort(v.begin(), v.end(), [](const std::string & a, const std::string & b) {
        std::string sa, sb;
        uint64_t ia = 0, ib = 0;
        if (trailing_index(a, &sa, &ia) && trailing_index(b, &sb, &ib) && sa == sb) return ia < ib;
        return a < b;
    });
    return v;
}

// IEEE binary16 -> binary32, exact (written out so the host compiler needs no
// half type).
static float half_to_float(uint16_t h) {
    const uint32_t sign = (uint32_t)(h >> 15) << 31;
    const uint32_t ex = (h >> 10) & 31, man = h & 1023;
    uint32_t u;
    if (ex == 0) {
        // zero or subnormal: man * 2^-24 (exact in fp32)
        float v = (float)man * 5.9604644775390625e-08f;
        std::memcpy(&u, &v, 4);
        u |= sign;
    } else if (ex == 31) {
        u = sign | 0x7f800000u | (man << 13);  // inf / nan
    } else {
        u = sign | ((ex + 112) << 23) | (man << 13);
    }
    float out;
    std::memcpy(&out, &u, 4);
    return out;
}

const float * payload_f32(const MappedFile & f, const TensorInfo & t, std::vector<float> & tmp) {
    if (t.offset + t.nbytes > f.size() || (t.nbytes == 0 && t.type != kF32))
        throw std::runtime_error("unsupported or truncated gguf tensor: " + t.name);
    if (t.type == kF32) return reinterpret_cast<const float *>(f.data() + t.offset);
    const size_t n = t.nbytes / 2;
    tmp.resize(n);
    const unsigned char * p = f.data() + t.offset;
    for (size_t i = 0; i < n; ++i) {
        uint16_t h;
        std::memcpy(&h, p + 2 * i, 2);
        if (t.type == kF16) {
            tmp[i] = half_to_float(h);
        } else {
            const uint32_t u = (uint32_t)h << 16;  // bf16 is the top half of an fp32
            std::memcpy(&tmp[i], &u, 4);
        }
    }
    return tmp.data();
}

}  // namespace gguf
}  // namespace sana
