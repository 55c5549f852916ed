// Byte-level BPE tokenizer over the GGUF vocabulary and merges (host).
//
// The reference builds a HuggingFace `tokenizers` (0.21.4, Cargo.lock) BPE
// from tokenizer.ggml.tokens and tokenizer.ggml.merges, with unk token
// "<unk>", a ByteLevel pre-tokenizer (add_prefix_space false, trim_offsets
// true, use_regex false: the whole text is one word, its bytes mapped to the
// GPT-2 alphabet) and a ByteLevel decoder (tokenizer.rs:22-90).  This class
// restates that library's published algorithm:
//  - encode: each byte of the text becomes the symbol of its alphabet
//    character (an unknown character becomes "<unk>", or the encode fails
//    when "<unk>" is not in the vocabulary); then every adjacent pair that
//    has a merge is queued by (rank, position), and the lowest rank, leftmost
//    first, is merged repeatedly (models/bpe/word.rs merge_all), entries made
//    stale by an earlier merge being skipped;
//  - merges: "a b" split at the first space; merge i has rank i and yields
//    the token a+b; a merge whose parts or result are not in the vocabulary
//    fails the build (a later duplicate pair overrides an earlier one);
//  - decode: each token's characters map back to bytes (a token with a
//    character outside the alphabet contributes its own UTF-8 bytes), and the
//    bytes are read as UTF-8 with every maximal invalid subsequence replaced
//    by U+FFFD (Rust's from_utf8_lossy).  Tokens such as "<|eot_id|>" are
//    ordinary vocabulary entries here, so they decode to their own text and
//    text containing them is encoded byte by byte like any other.
// The chat templates and stop ids follow tokenizer.rs:160-216.
#pragma once

#include <cstdint>
#include <string>
#include <unordered_map>
#include <vector>

#include "gguf.h"

namespace oxb {

struct ChatMsg {
    std::string role, content;
};

class Tokenizer {
  public:
    // false + thread error ("Tokenizer error: ...") on a missing vocabulary
    // or a merge the vocabulary cannot hold
    bool init(const GgufFile &g);
    // false + thread error when a character has no symbol and "<unk>" is
    // not in the vocabulary
    bool encode(const std::string &text, bool add_bos, std::vector<int32_t> &out) const;
    std::string decode_one(int32_t id) const;
    bool apply_chat_template(const std::vector<ChatMsg> &msgs, std::vector<int32_t> &out) const;
    int32_t bos() const { return bos_; }
    int32_t eos() const { return eos_; }
    int32_t eot() const { return eot_; }      // -1 if absent
    int32_t im_end() const { return im_end_; }
    int32_t id_of(const std::string &tok) const;
    size_t vocab_size() const { return vocab_.size(); }

  private:
    std::vector<std::string> vocab_;
    std::unordered_map<std::string, int32_t> ids_;
    // (left id << 32 | right id) -> (rank, merged id)
    std::unordered_map<uint64_t, std::pair<int32_t, int32_t>> merges_;
    int32_t byte_id_[256];   // vocabulary id of each byte's alphabet character, -1 if none
    int32_t unk_ = -1;
    int32_t bos_ = 1, eos_ = 2, eot_ = -1, im_end_ = -1;
    std::string byte_enc_[256];
    std::unordered_map<uint32_t, uint8_t> byte_dec_;
};

}  // namespace oxb
