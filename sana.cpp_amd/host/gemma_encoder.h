// Drop-in Gemma-2 prompt encoder: the declarations of the reference's
// src/gemma_encoder.h:14-48, with the decoder forward on the HIP gfx950 path
// (sana_gemma_* of include/sana_dit.h) instead of llama.cpp, and a
// SentencePiece-BPE tokenizer read from the GGUF's tokenizer metadata.
#pragma once

#include <cstdint>
#include <memory>
#include <string>
#include <vector>

#include "tensor.h"

struct GemmaEncoderConfig {
    std::string gguf_path;
    size_t max_sequence_length = 300;
    int32_t n_threads = 4;  // kept for source compatibility; the forward runs on the GPU
};

// Owns the device model and the tokenizer, so one process can encode many
// prompts without reloading the GGUF.
struct GemmaEncoder {
    explicit GemmaEncoder(const GemmaEncoderConfig & config);
    ~GemmaEncoder();
    GemmaEncoder(const GemmaEncoder &) = delete;
    GemmaEncoder & operator=(const GemmaEncoder &) = delete;

    struct Impl;
    std::unique_ptr<Impl> impl;
};

// Batch order as diffusers: the negative prompt first, then the positive one.
struct GemmaPromptPair {
    Tensor embeddings;      // (2, max_sequence_length, hidden_size)
    Tensor attention_bias;  // (2, 1, max_sequence_length), (1 - mask) * -10000.0
};

GemmaPromptPair encode_prompt_pair(GemmaEncoder & encoder, const std::string & prompt,
                                   const std::string & negative_prompt, size_t max_sequence_length = 300);

// Row 0 and the last keep - 1 rows: select_index = [0] + [-(keep-1), ..., -1].
Tensor select_rows_first_and_last(const Tensor & input, size_t keep);

// Token ids of `text` as the encoder tokenizes it: the BOS token (when the
// vocabulary adds one), special tokens matched in the text, the rest by
// score-ordered BPE merges with byte fallback.
std::vector<int32_t> gemma_tokenize(const GemmaEncoder & encoder, const std::string & text);

// The same for the tokenizer of a GGUF file alone (no device model).
std::vector<int32_t> gemma_tokenize_gguf(const std::string & gguf_path, const std::string & text);
