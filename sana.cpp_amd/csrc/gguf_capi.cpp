// GGUF entry points of the C ABI: sana_dit_load_gguf (the three-file loader of
// load_denoiser_weights, src/transformer.cpp:453-488) and the index
// inspection helpers.
#include <sys/stat.h>

#include <cstdio>
#include <cstring>
#include <map>
#include <memory>
#include <mutex>
#include <stdexcept>
#include <string>
#include <vector>

#include "../../include/sana_dit.h"
#include "gguf.h"

namespace sana {
void set_last_error(const std::string & m);  // dit.hip: storage behind sana_dit_last_error()
}

namespace {

// Block tensors the reference loads per prefix (src/transformer.cpp:214-308).
const char * const kBlockSuffixes[] = {
    "scale_shift_table", "attn1.to_q.weight", "attn1.to_k.weight", "attn1.to_v.weight", "attn1.to_out.0.weight",
    "attn1.to_out.0.bias", "attn2.to_q.weight", "attn2.to_q.bias", "attn2.to_k.weight", "attn2.to_k.bias",
    "attn2.to_v.weight", "attn2.to_v.bias", "attn2.to_out.0.weight", "attn2.to_out.0.bias",
    "ff.conv_inverted.weight", "ff.conv_inverted.bias", "ff.conv_depth.weight", "ff.conv_depth.bias",
    "ff.conv_point.weight",
};
const char * const kCaptionNames[] = {
    "caption_projection.linear_1.weight", "caption_projection.linear_1.bias", "caption_projection.linear_2.weight",
    "caption_projection.linear_2.bias",
};
const char * const kDenoiserNames[] = {
    "patch_embed.proj.weight", "patch_embed.proj.bias", "time_embed.emb.timestep_embedder.linear_1.weight",
    "time_embed.emb.timestep_embedder.linear_1.bias", "time_embed.emb.timestep_embedder.linear_2.weight",
    "time_embed.emb.timestep_embedder.linear_2.bias", "time_embed.linear.weight", "time_embed.linear.bias",
    "caption_norm.weight", "scale_shift_table", "proj_out.weight", "proj_out.bias",
};


struct Err {
    int code;
    std::string msg;
};

// F32 payloads are read in place; F16 and BF16 are widened to fp32 first (the
// reference reads every payload as raw F32 whatever its ggml type,
// src/weights_io.cpp:155, :340-355, which misreads 16-bit files).  Other types
// are refused.
const float * payload(const sana::gguf::MappedFile & f, const sana::gguf::TensorInfo & t, std::vector<float> & tmp) {
    using namespace sana::gguf;
    if (t.type != kF32 && t.type != kF16 && t.type != kBF16)
        throw Err{SANA_ERR_FORMAT, "gguf tensor type must be F32, F16 or BF16: " + t.name};
    try {
        return payload_f32(f, t, tmp);
    } catch (const std::runtime_error & e) {
        throw Err{SANA_ERR_FORMAT, e.what()};
    }
}

// Linear weights held as fp16 GEMM operands on the device: an F16 payload of
// one of these is copied as stored (sana_dit_set_*_f16).
bool is_block_operand(const std::string & s) {
    static const char * const k[] = {"attn1.to_q.weight", "attn1.to_k.weight",     "attn1.to_v.weight",
                                     "attn1.to_out.0.weight", "attn2.to_q.weight", "attn2.to_k.weight",
                                     "attn2.to_v.weight", "attn2.to_out.0.weight", "ff.conv_inverted.weight",
                                     "ff.conv_point.weight"};
    for (const char * n : k)
        if (s == n) return true;
    return false;
}
bool is_top_operand(const std::string & s) {
    return s == "caption_projection.linear_1.weight" || s == "caption_projection.linear_2.weight";
}

// The F16 payload in place (bounds checked against the mapping).
const uint16_t * f16_payload(const sana::gguf::MappedFile & f, const sana::gguf::TensorInfo & t) {
    if (t.offset + t.nbytes > f.size() || t.nbytes == 0 || (t.offset & 1))
        throw Err{SANA_ERR_FORMAT, "unsupported or truncated gguf tensor: " + t.name};
    return reinterpret_cast<const uint16_t *>(f.data() + t.offset);
}

const sana::gguf::TensorInfo & find(const sana::gguf::Index & idx, const std::string & n) {
    for (const auto & t : idx.tensors)
        if (t.name == n) return t;
    throw Err{SANA_ERR_INVALID_ARGUMENT, "weight name not found in weight index: " + n};
}

void call(int rc) {
    if (rc != SANA_OK) throw Err{rc, sana_dit_last_error()};
}

// Small cache so the per-index inspection calls do not re-parse the file.
std::mutex g_cache_mu;
std::string g_cache_path;
std::shared_ptr<sana::gguf::Index> g_cache;

std::shared_ptr<sana::gguf::Index> cached_index(const std::string & path) {
    std::lock_guard<std::mutex> lk(g_cache_mu);
    if (!g_cache || g_cache_path != path) {
        g_cache = std::make_shared<sana::gguf::Index>(sana::gguf::read_index(path));
        g_cache_path = path;
    }
    return g_cache;
}

// Key of a set of source files: FNV-1a over each path, size, modification
// time and first MiB (the GGUF header and tensor directory).
uint64_t source_key(const char * const * paths, int n) {
    uint64_t h = 14695981039346656037ULL;
    auto mix = [&](const void * p, size_t len) {
        const unsigned char * b = static_cast<const unsigned char *>(p);
        for (size_t i = 0; i < len; ++i) h = (h ^ b[i]) * 1099511628211ULL;
    };
    std::vector<unsigned char> head(1u << 20);
    for (int i = 0; i < n; ++i) {
        struct stat st;
        if (stat(paths[i], &st) != 0) throw Err{SANA_ERR_IO, std::string("cannot stat ") + paths[i]};
        mix(paths[i], std::strlen(paths[i]) + 1);
        const int64_t meta[3] = {(int64_t)st.st_size, (int64_t)st.st_mtim.tv_sec, (int64_t)st.st_mtim.tv_nsec};
        mix(meta, sizeof(meta));
        FILE * f = std::fopen(paths[i], "rb");
        if (!f) throw Err{SANA_ERR_IO, std::string("cannot open ") + paths[i]};
        const size_t got = std::fread(head.data(), 1, head.size(), f);
        std::fclose(f);
        mix(head.data(), got);
    }
    return h;
}

template <class F>
int guarded(F f) {
    try {
        f();
        return SANA_OK;
    } catch (const Err & e) {
        sana::set_last_error(e.msg);
        return e.code;
    } catch (const std::exception & e) {
        sana::set_last_error(e.what());
        return SANA_ERR_IO;
    }
}

}  // namespace

extern "C" {

int sana_dit_load_gguf(sana_dit * ctx, const char * model_path, const char * caption_path, const char * denoiser_path) {
    if (!ctx || !model_path || !caption_path || !denoiser_path) {
        sana::set_last_error("null argument");
        return SANA_ERR_INVALID_ARGUMENT;
    }
    return guarded([&] {
        using namespace sana::gguf;
        // model blocks
        {
            const Index idx = read_index(model_path);
            MappedFile f(model_path);
            std::vector<std::string> names;
            for (const auto & t : idx.tensors) names.push_back(t.name);
            const std::vector<std::string> pre = block_prefixes(names);
            std::vector<float> tmp;
            if (pre.empty()) throw Err{SANA_ERR_INVALID_ARGUMENT, "weight index does not contain any prefixed model blocks"};
            for (size_t b = 0; b < pre.size(); ++b) {
                for (const char * s : kBlockSuffixes) {
                    const std::string full = pre[b].empty() ? std::string(s) : pre[b] + "." + s;
                    const TensorInfo & t = find(idx, full);
                    int rc = t.type == kF16 && is_block_operand(s)
                                 ? sana_dit_set_block_weight_f16(ctx, (int64_t)b, s, f16_payload(f, t), t.shape.data(),
                                                                 (int)t.shape.size())
                                 : sana_dit_set_block_weight(ctx, (int64_t)b, s, payload(f, t, tmp), t.shape.data(),
                                                             (int)t.shape.size(), 0);
                    if (rc == SANA_ERR_INVALID_ARGUMENT && b > 0)
                        throw Err{SANA_ERR_SHAPE, "gguf holds more blocks than the model's layer count"};
                    call(rc);
                }
            }
        }
        for (int which = 0; which < 2; ++which) {
            const char * path = which == 0 ? caption_path : denoiser_path;
            const Index idx = read_index(path);
            MappedFile f(path);
            std::vector<float> tmp;
            const size_t n = which == 0 ? sizeof(kCaptionNames) / sizeof(kCaptionNames[0])
                                        : sizeof(kDenoiserNames) / sizeof(kDenoiserNames[0]);
            for (size_t i = 0; i < n; ++i) {
                const char * name = which == 0 ? kCaptionNames[i] : kDenoiserNames[i];
                const TensorInfo & t = find(idx, name);
                if (t.type == kF16 && is_top_operand(name))
                    call(sana_dit_set_weight_f16(ctx, name, f16_payload(f, t), t.shape.data(), (int)t.shape.size()));
                else
                    call(sana_dit_set_weight(ctx, name, payload(f, t, tmp), t.shape.data(), (int)t.shape.size(), 0));
            }
        }
        call(sana_dit_check_weights(ctx));
    });
}

int sana_dit_load_gguf_cached(sana_dit * ctx, const char * model_path, const char * caption_path,
                              const char * denoiser_path, const char * cache_path, int * used_cache) {
    if (used_cache) *used_cache = 0;
    if (!ctx || !model_path || !caption_path || !denoiser_path || !cache_path) {
        sana::set_last_error("null argument");
        return SANA_ERR_INVALID_ARGUMENT;
    }
    uint64_t key = 0;
    const char * const paths[3] = {model_path, caption_path, denoiser_path};
    int rc = guarded([&] { key = source_key(paths, 3); });
    if (rc != SANA_OK) return rc;
    if (sana_dit_load_packed(ctx, cache_path, key) == SANA_OK) {
        if (used_cache) *used_cache = 1;
        return SANA_OK;
    }
    rc = sana_dit_load_gguf(ctx, model_path, caption_path, denoiser_path);
    if (rc != SANA_OK) return rc;
    (void)sana_dit_save_packed(ctx, cache_path, key);  // best effort
    return SANA_OK;
}

int sana_gguf_num_tensors(const char * path, int64_t * n) {
    if (!path || !n) {
        sana::set_last_error("null argument");
        return SANA_ERR_INVALID_ARGUMENT;
    }
    return guarded([&] { *n = (int64_t)cached_index(path)->tensors.size(); });
}

int sana_gguf_tensor_info(const char * path, int64_t i, char * name, size_t name_cap, int64_t * shape, int * ndim,
                          int * type, uint64_t * offset) {
    if (!path || !name || !shape || !ndim || !type || !offset) {
        sana::set_last_error("null argument");
        return SANA_ERR_INVALID_ARGUMENT;
    }
    return guarded([&] {
        auto idx = cached_index(path);
        if (i < 0 || i >= (int64_t)idx->tensors.size()) throw Err{SANA_ERR_INVALID_ARGUMENT, "tensor index out of range"};
        const auto & t = idx->tensors[i];
        if (t.name.size() + 1 > name_cap) throw Err{SANA_ERR_INVALID_ARGUMENT, "name buffer too small"};
        std::memcpy(name, t.name.c_str(), t.name.size() + 1);
        *ndim = (int)t.shape.size();
        for (size_t d = 0; d < t.shape.size(); ++d) shape[d] = t.shape[d];
        *type = (int)t.type;
        *offset = t.offset;
    });
}

}  // extern "C"
