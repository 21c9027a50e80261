// Drop-in Gemma-2 prompt encoder on the HIP gfx950 path.
//
// The reference tokenizes with llama.cpp's SentencePiece (SPM) tokenizer and
// runs the model with llama_decode in embeddings mode (src/gemma_encoder.cpp:
// 27-152). Here:
// - the model hyperparameters and the vocabulary come from the GGUF metadata
//   that llama.cpp reads: {arch}.embedding_length, block_count,
//   feed_forward_length, attention.*, rope.freq_base, attn_logit_softcapping,
//   and tokenizer.ggml.*;
// - the tokenizer is written from the published SentencePiece-BPE procedure:
//   special tokens matched in the text first, spaces escaped to U+2581, then
//   adjacent symbols merged highest score first (the leftmost pair on a tie)
//   while the merged text is a vocabulary piece, and the pieces still outside
//   the vocabulary emitted as <0xXX> byte tokens;
// - the forward runs on the device (sana_gemma_* in include/sana_dit.h).
// encode_prompt_pair, select_rows_first_and_last and the padding-mask bias
// follow the reference's steps (src/gemma_encoder.cpp:53-244).
#include "gemma_encoder.h"

#include <algorithm>
#include <cmath>
#include <cstdlib>
#include <queue>
#include <stdexcept>
#include <unordered_map>
#include <utility>

#include "../../include/sana_dit.h"
#include "../csrc/gguf.h"

namespace {

[[noreturn]] void raise_abi(int rc) {
    const std::string msg = sana_dit_last_error();
    if (rc == SANA_ERR_INVALID_ARGUMENT || rc == SANA_ERR_SHAPE) throw std::invalid_argument(msg);
    throw std::runtime_error(msg);
}

void ck(int rc) {
    if (rc != SANA_OK) raise_abi(rc);
}

// The instruction prefix diffusers' SanaPipeline puts in front of the
// positive prompt (complex_human_instruction), as the reference uses it.
const char * const kComplexHumanInstruction =
    "Given a user prompt, generate an 'Enhanced prompt' that provides detailed visual descriptions suitable for "
    "image generation. Evaluate the level of detail in the user prompt:\n"
    "- If the prompt is simple, focus on adding specifics about colors, shapes, sizes, textures, and spatial "
    "relationships to create vivid and concrete scenes.\n"
    "- If the prompt is already detailed, refine and enhance the existing details slightly without "
    "overcomplicating.\n"
    "Here are examples of how to transform or refine prompts:\n"
    "- User Prompt: A cat sleeping -> Enhanced: A small, fluffy white cat curled up in a round shape, sleeping "
    "peacefully on a warm sunny windowsill, surrounded by pots of blooming red flowers.\n"
    "- User Prompt: A busy city street -> Enhanced: A bustling city street scene at dusk, featuring glowing street "
    "lamps, a diverse crowd of people in colorful clothing, and a double-decker bus passing by towering glass "
    "skyscrapers.\n"
    "Please generate only the enhanced description for the prompt below and avoid including any additional "
    "commentary or evaluations:\n"
    "User Prompt: ";

// GGUF token types (tokenizer.ggml.token_type).
enum TokenType { kNormal = 1, kUnknown = 2, kControl = 3, kUserDefined = 4, kUnused = 5, kByte = 6 };

struct SpmTokenizer {
    std::vector<std::string> text;
    std::vector<float> score;
    std::vector<int> type;
    std::unordered_map<std::string, int32_t> id;
    std::vector<int32_t> special;  // matched in the text, longest first
    int32_t byte_id[256];
    int32_t bos = -1;
    bool add_bos = true, add_space_prefix = false;

    void bpe(const std::string & s, std::vector<int32_t> & out) const;
    std::vector<int32_t> encode(const std::string & s) const;
};

size_t utf8_len(unsigned char c) {
    static const size_t len[16] = {1, 1, 1, 1, 1, 1, 1, 1, 1, 1, 1, 1, 2, 2, 3, 4};
    return len[c >> 4];
}

void SpmTokenizer::bpe(const std::string & s, std::vector<int32_t> & out) const {
    struct Sym {
        int prev, next;
        size_t pos, len;
    };
    struct Pair {
        int left, right;
        float score;
        size_t len;
    };
    // highest score first; on a tie the leftmost pair
    auto worse = [](const Pair & a, const Pair & b) {
        return a.score < b.score || (a.score == b.score && a.left > b.left);
    };
    std::vector<Sym> sym;
    for (size_t pos = 0; pos < s.size();) {
        const size_t len = std::min(utf8_len(static_cast<unsigned char>(s[pos])), s.size() - pos);
        const int i = (int)sym.size();
        sym.push_back(Sym{i - 1, -1, pos, len});
        if (i > 0) sym[i - 1].next = i;
        pos += len;
    }
    std::priority_queue<Pair, std::vector<Pair>, decltype(worse)> q(worse);
    auto try_pair = [&](int l, int r) {
        if (l < 0 || r < 0) return;
        const auto it = id.find(s.substr(sym[l].pos, sym[l].len + sym[r].len));
        if (it == id.end()) return;
        q.push(Pair{l, r, score[it->second], sym[l].len + sym[r].len});
    };
    for (int i = 0; i + 1 < (int)sym.size(); ++i) try_pair(i, i + 1);
    while (!q.empty()) {
        const Pair p = q.top();
        q.pop();
        Sym & l = sym[p.left];
        Sym & r = sym[p.right];
        if (l.len == 0 || r.len == 0 || l.len + r.len != p.len) continue;  // stale pair
        l.len += r.len;
        r.len = 0;
        l.next = r.next;
        if (r.next >= 0) sym[r.next].prev = p.left;
        try_pair(l.prev, p.left);
        try_pair(p.left, l.next);
    }
    for (int i = sym.empty() ? -1 : 0; i >= 0; i = sym[i].next) {
        const std::string piece = s.substr(sym[i].pos, sym[i].len);
        const auto it = id.find(piece);
        if (it != id.end()) {
            out.push_back(it->second);
        } else {
            for (unsigned char c : piece) {
                if (byte_id[c] < 0) throw std::runtime_error("tokenizer has no byte token for a byte of the input");
                out.push_back(byte_id[c]);
            }
        }
    }
}

std::vector<int32_t> SpmTokenizer::encode(const std::string & s) const {
    // split out the special tokens (longest first), then BPE the rest
    struct Frag {
        int32_t token;  // -1: raw text
        std::string raw;
    };
    std::vector<Frag> frags{Frag{-1, s}};
    for (int32_t sid : special) {
        const std::string & st = text[sid];
        if (st.empty()) continue;
        std::vector<Frag> next;
        for (Frag & f : frags) {
            if (f.token >= 0) {
                next.push_back(std::move(f));
                continue;
            }
            size_t from = 0;
            for (size_t at; (at = f.raw.find(st, from)) != std::string::npos; from = at + st.size()) {
                if (at > from) next.push_back(Frag{-1, f.raw.substr(from, at - from)});
                next.push_back(Frag{sid, std::string()});
            }
            if (from < f.raw.size()) next.push_back(Frag{-1, f.raw.substr(from)});
        }
        frags.swap(next);
    }
    std::vector<int32_t> out;
    bool prev_special = true;
    if (add_bos && bos >= 0) out.push_back(bos);
    for (const Frag & f : frags) {
        if (f.token >= 0) {
            out.push_back(f.token);
            prev_special = true;
            continue;
        }
        const std::string t = (add_space_prefix && prev_special) ? " " + f.raw : f.raw;
        std::string esc;
        for (char c : t) {
            if (c == ' ') esc += "\xE2\x96\x81";  // U+2581
            else esc += c;
        }
        bpe(esc, out);
        prev_special = false;
    }
    return out;
}

const sana::gguf::MetaValue * meta(const sana::gguf::Index & idx, const std::string & key) {
    const auto it = idx.meta.find(key);
    return it == idx.meta.end() ? nullptr : &it->second;
}

double meta_num(const sana::gguf::Index & idx, const std::string & key, double fallback, bool required = false) {
    const sana::gguf::MetaValue * v = meta(idx, key);
    if (!v || v->type == 8 || v->type == 9) {  // string, array
        if (required) throw std::runtime_error("gguf metadata key missing or not a number: " + key);
        return fallback;
    }
    return v->num;
}

SpmTokenizer load_tokenizer(const sana::gguf::Index & idx) {
    SpmTokenizer t;
    const sana::gguf::MetaValue * model = meta(idx, "tokenizer.ggml.model");
    if (!model || model->str != "llama")
        throw std::runtime_error("gguf tokenizer must be tokenizer.ggml.model = llama (SentencePiece): " + idx.path);
    const sana::gguf::MetaValue * toks = meta(idx, "tokenizer.ggml.tokens");
    if (!toks || toks->strs.empty()) throw std::runtime_error("gguf has no tokenizer.ggml.tokens: " + idx.path);
    t.text = toks->strs;
    const size_t n = t.text.size();
    const sana::gguf::MetaValue * sc = meta(idx, "tokenizer.ggml.scores");
    const sana::gguf::MetaValue * ty = meta(idx, "tokenizer.ggml.token_type");
    t.score.assign(n, 0.0f);
    t.type.assign(n, kNormal);
    if (sc && sc->nums.size() == n)
        for (size_t i = 0; i < n; ++i) t.score[i] = (float)sc->nums[i];
    if (ty && ty->nums.size() == n)
        for (size_t i = 0; i < n; ++i) t.type[i] = (int)ty->nums[i];
    std::fill(std::begin(t.byte_id), std::end(t.byte_id), -1);
    for (size_t i = 0; i < n; ++i) {
        t.id.emplace(t.text[i], (int32_t)i);
        if (t.type[i] == kByte && t.text[i].size() == 6 && t.text[i].compare(0, 3, "<0x") == 0) {
            const long b = std::strtol(t.text[i].substr(3, 2).c_str(), nullptr, 16);
            if (b >= 0 && b < 256) t.byte_id[b] = (int32_t)i;
        }
        if (t.type[i] == kControl || t.type[i] == kUserDefined || t.type[i] == kUnknown)
            t.special.push_back((int32_t)i);
    }
    std::stable_sort(t.special.begin(), t.special.end(),
                     [&](int32_t a, int32_t b) { return t.text[a].size() > t.text[b].size(); });
    t.bos = (int32_t)meta_num(idx, "tokenizer.ggml.bos_token_id", -1);
    t.add_bos = meta_num(idx, "tokenizer.ggml.add_bos_token", 1) != 0;
    t.add_space_prefix = meta_num(idx, "tokenizer.ggml.add_space_prefix", 1) != 0;
    return t;
}

}  // namespace

struct GemmaEncoder::Impl {
    sana_gemma * model = nullptr;
    SpmTokenizer tok;
    int64_t hidden = 0;

    explicit Impl(const GemmaEncoderConfig & config) {
        sana::gguf::Index idx;
        try {
            idx = sana::gguf::read_index(config.gguf_path);
        } catch (const std::exception & e) {
            throw std::runtime_error("failed to load Gemma-2 GGUF: " + config.gguf_path + " (" + e.what() + ")");
        }
        const sana::gguf::MetaValue * a = meta(idx, "general.architecture");
        const std::string arch = a ? a->str : "gemma2";
        tok = load_tokenizer(idx);
        sana_gemma_config c{};
        c.vocab = (int64_t)tok.text.size();
        c.hidden = (int64_t)meta_num(idx, arch + ".embedding_length", 0, true);
        c.layers = (int64_t)meta_num(idx, arch + ".block_count", 0, true);
        c.ffn = (int64_t)meta_num(idx, arch + ".feed_forward_length", 0, true);
        c.heads = (int64_t)meta_num(idx, arch + ".attention.head_count", 0, true);
        c.kv_heads = (int64_t)meta_num(idx, arch + ".attention.head_count_kv", (double)c.heads);
        c.head_dim =
            (int64_t)meta_num(idx, arch + ".attention.key_length", c.heads ? (double)(c.hidden / c.heads) : 0.0);
        c.rms_eps = (float)meta_num(idx, arch + ".attention.layer_norm_rms_epsilon", 1e-6);
        c.sliding_window = (int64_t)meta_num(idx, arch + ".attention.sliding_window", 0);
        c.attn_softcap = (float)meta_num(idx, arch + ".attn_logit_softcapping", 50.0);
        c.rope_theta = (float)meta_num(idx, arch + ".rope.freq_base", 10000.0);
        c.query_scale = c.head_dim > 0 ? 1.0f / std::sqrt((float)c.head_dim) : 0.0f;
        const char * e = std::getenv("SANA_HIP_DEVICE");
        c.device = e ? std::atoi(e) : 0;
        hidden = c.hidden;
        ck(sana_gemma_create(&c, &model));
        const int rc = sana_gemma_load_gguf(model, config.gguf_path.c_str());
        if (rc != SANA_OK) {
            const std::string msg = sana_dit_last_error();
            sana_gemma_destroy(model);
            model = nullptr;
            throw std::runtime_error("failed to load Gemma-2 GGUF: " + config.gguf_path + " (" + msg + ")");
        }
    }

    ~Impl() {
        if (model) sana_gemma_destroy(model);
    }

    // Per-token hidden states after the final norm, (n_tokens, hidden).
    Tensor decode_embeddings(const std::vector<int32_t> & tokens) {
        Tensor out({tokens.size(), static_cast<size_t>(hidden)});
        ck(sana_gemma_encode(model, tokens.data(), (int64_t)tokens.size(), out.data().data()));
        return out;
    }

    // Both sequences in one device pass; the same values as two
    // decode_embeddings calls.
    std::pair<Tensor, Tensor> decode_embeddings_pair(const std::vector<int32_t> & a, const std::vector<int32_t> & b) {
        Tensor oa({a.size(), static_cast<size_t>(hidden)}), ob({b.size(), static_cast<size_t>(hidden)});
        ck(sana_gemma_encode_pair(model, a.data(), (int64_t)a.size(), b.data(), (int64_t)b.size(),
                                  oa.data().data(), ob.data().data()));
        return {std::move(oa), std::move(ob)};
    }
};

GemmaEncoder::GemmaEncoder(const GemmaEncoderConfig & config) : impl(std::make_unique<Impl>(config)) {}

GemmaEncoder::~GemmaEncoder() = default;

std::vector<int32_t> gemma_tokenize(const GemmaEncoder & encoder, const std::string & text) {
    return encoder.impl->tok.encode(text);
}

std::vector<int32_t> gemma_tokenize_gguf(const std::string & gguf_path, const std::string & text) {
    return load_tokenizer(sana::gguf::read_index(gguf_path)).encode(text);
}

Tensor select_rows_first_and_last(const Tensor & input, size_t keep) {
    if (input.rank() != 2) throw std::invalid_argument("select_rows_first_and_last expects a rank-2 tensor");
    const size_t rows = input.dim_size(0), cols = input.dim_size(1);
    if (keep == 0 || keep > rows) throw std::invalid_argument("select_rows_first_and_last: keep must be in (0, rows]");
    Tensor out({keep, cols});
    const float * src = input.data().data();
    float * dst = out.data().data();
    std::copy(src, src + cols, dst);
    std::copy(src + (rows - (keep - 1)) * cols, src + rows * cols, dst + cols);
    return out;
}

namespace {

struct Padded {
    std::vector<int32_t> tokens;
    size_t real = 0;
};

Padded tokenize_padded(const SpmTokenizer & tok, const std::string & text, size_t length) {
    Padded p;
    p.tokens = tok.encode(text);
    if (p.tokens.size() > length)
        throw std::invalid_argument("tokenized text exceeds padded_length; truncation not implemented");
    p.real = p.tokens.size();
    p.tokens.resize(length, 0);  // pad id 0
    return p;
}

void write_bias(Tensor & bias, size_t row, size_t real, size_t length) {
    float * d = bias.data().data() + row * length;
    for (size_t t = 0; t < length; ++t) d[t] = t < real ? 0.0f : -10000.0f;
}

}  // namespace

GemmaPromptPair encode_prompt_pair(GemmaEncoder & encoder, const std::string & prompt,
                                   const std::string & negative_prompt, size_t max_sequence_length) {
    GemmaEncoder::Impl & m = *encoder.impl;
    const size_t H = static_cast<size_t>(m.hidden), L = max_sequence_length;
    if (L < 2) throw std::invalid_argument("max_sequence_length must be at least 2");
    // positive: instruction + prompt, padded to len(instruction tokens) + L - 2,
    // then row 0 and the last L - 1 rows
    const size_t chi = m.tok.encode(kComplexHumanInstruction).size();
    const size_t all = chi + L - 2;
    const Padded pos = tokenize_padded(m.tok, std::string(kComplexHumanInstruction) + prompt, all);
    size_t pos_real = pos.real > 0 ? 1 : 0;  // row 0 (BOS)
    for (size_t p = all - (L - 1); p < all; ++p)
        if (p < pos.real) ++pos_real;
    // negative: no instruction, padded to L, no selection
    const Padded neg = tokenize_padded(m.tok, negative_prompt, L);
    // both prompts through the encoder in one pass
    std::pair<Tensor, Tensor> emb = m.decode_embeddings_pair(pos.tokens, neg.tokens);
    const Tensor pos_sel = select_rows_first_and_last(emb.first, L);
    const Tensor & neg_emb = emb.second;
    GemmaPromptPair r{Tensor({2, L, H}), Tensor({2, 1, L})};
    std::copy(neg_emb.data().begin(), neg_emb.data().end(), r.embeddings.data().begin());
    std::copy(pos_sel.data().begin(), pos_sel.data().end(), r.embeddings.data().begin() + L * H);
    write_bias(r.attention_bias, 0, neg.real, L);
    write_bias(r.attention_bias, 1, pos_real, L);
    return r;
}
