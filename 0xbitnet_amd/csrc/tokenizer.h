// Minimal byte-level tokenizer over the GGUF vocabulary (host).
//
// The reference builds a HF `tokenizers` BPE from tokenizer.ggml.tokens and
// .merges with a GPT-2 byte-level pre-tokenizer (tokenizer.rs:22-90).  This
// build's scope is the ternary inference path, so text handling is a
// pass-through: the same GPT-2 byte <-> unicode mapping, greedy longest match
// over the vocabulary instead of merge ranks (ids can differ from the BPE's
// on text the merges would split differently), the same special tokens, the
// same chat templates (tokenizer.rs:160-216) and the same stop ids.
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
    // false + thread error "Tokenizer error: Missing tokenizer.ggml.tokens"
    bool init(const GgufFile &g);
    std::vector<int32_t> encode(const std::string &text, bool add_bos) const;
    std::string decode_one(int32_t id) const;
    std::vector<int32_t> apply_chat_template(const std::vector<ChatMsg> &msgs) const;
    int32_t bos() const { return bos_; }
    int32_t eos() const { return eos_; }
    int32_t eot() const { return eot_; }      // -1 if absent
    int32_t im_end() const { return im_end_; }
    int32_t id_of(const std::string &tok) const;

  private:
    std::vector<std::string> vocab_;
    std::unordered_map<std::string, int32_t> ids_;
    std::vector<std::string> specials_;  // "<|...|>" tokens, matched verbatim
    size_t max_len_ = 1;
    int32_t bos_ = 1, eos_ = 2, eot_ = -1, im_end_ = -1;
    std::string byte_enc_[256];
    std::unordered_map<uint32_t, uint8_t> byte_dec_;
};

}  // namespace oxb
