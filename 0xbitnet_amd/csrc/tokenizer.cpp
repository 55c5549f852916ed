// See tokenizer.h.
#include "tokenizer.h"

#include <cstring>

#include "oxb_common.h"

namespace oxb {

namespace {

void put_utf8(std::string &s, uint32_t cp) {
    if (cp < 0x80) {
        s += (char)cp;
    } else if (cp < 0x800) {
        s += (char)(0xC0 | (cp >> 6));
        s += (char)(0x80 | (cp & 0x3F));
    } else {
        s += (char)(0xE0 | (cp >> 12));
        s += (char)(0x80 | ((cp >> 6) & 0x3F));
        s += (char)(0x80 | (cp & 0x3F));
    }
}

// Next code point of a UTF-8 string (invalid bytes are returned as is).
uint32_t next_cp(const std::string &s, size_t &i) {
    const uint8_t c = (uint8_t)s[i];
    int n = c < 0x80 ? 1 : (c >> 5) == 6 ? 2 : (c >> 4) == 14 ? 3 : (c >> 3) == 30 ? 4 : 1;
    if (i + n > s.size()) n = 1;
    uint32_t cp = n == 1 ? c : n == 2 ? (c & 0x1F) : n == 3 ? (c & 0x0F) : (c & 0x07);
    for (int k = 1; k < n; ++k) cp = (cp << 6) | ((uint8_t)s[i + k] & 0x3F);
    i += n;
    return cp;
}

}  // namespace

bool Tokenizer::init(const GgufFile &g) {
    const GgufValue *toks = g.get("tokenizer.ggml.tokens");
    if (!toks || toks->kind != GgufValue::ARR) {
        set_error("Tokenizer error: Missing tokenizer.ggml.tokens");
        return false;
    }
    vocab_.clear();
    ids_.clear();
    for (size_t i = 0; i < toks->arr.size(); ++i) {
        const std::string &t = toks->arr[i].s;
        vocab_.push_back(t);
        ids_.emplace(t, (int32_t)i);
        if (t.size() > max_len_) max_len_ = t.size();
        if (t.size() > 4 && t.compare(0, 2, "<|") == 0 && t.compare(t.size() - 2, 2, "|>") == 0)
            specials_.push_back(t);
    }
    if (auto *v = g.get("tokenizer.ggml.bos_token_id"); v && v->is_int()) bos_ = (int32_t)v->u;
    if (auto *v = g.get("tokenizer.ggml.eos_token_id"); v && v->is_int()) eos_ = (int32_t)v->u;
    eot_ = id_of("<|eot_id|>");
    im_end_ = id_of("<|im_end|>");
    // GPT-2 byte-level alphabet: printable bytes map to themselves, the rest
    // to U+0100 + n in byte order.
    int n = 0;
    for (int b = 0; b < 256; ++b) {
        const bool keep = (b >= 33 && b <= 126) || (b >= 161 && b <= 172) || (b >= 174 && b <= 255);
        const uint32_t cp = keep ? (uint32_t)b : (uint32_t)(256 + n++);
        byte_enc_[b].clear();
        put_utf8(byte_enc_[b], cp);
        byte_dec_[cp] = (uint8_t)b;
    }
    return true;
}

int32_t Tokenizer::id_of(const std::string &tok) const {
    auto it = ids_.find(tok);
    return it == ids_.end() ? -1 : it->second;
}

std::vector<int32_t> Tokenizer::encode(const std::string &text, bool add_bos) const {
    std::vector<int32_t> out;
    if (add_bos) out.push_back(bos_);
    std::string enc;
    for (unsigned char c : text) enc += byte_enc_[c];
    size_t i = 0;
    while (i < enc.size()) {
        size_t best = 0;
        int32_t best_id = -1;
        const size_t lim = std::min(max_len_, enc.size() - i);
        for (size_t len = lim; len > 0; --len) {
            auto it = ids_.find(enc.substr(i, len));
            if (it != ids_.end()) {
                best = len;
                best_id = it->second;
                break;
            }
        }
        if (best_id < 0) {  // no vocabulary entry starts here: skip one code point
            next_cp(enc, i);
            continue;
        }
        out.push_back(best_id);
        i += best;
    }
    return out;
}

std::string Tokenizer::decode_one(int32_t id) const {
    if (id < 0 || (size_t)id >= vocab_.size()) return std::string();
    const std::string &t = vocab_[id];
    if (t.size() > 4 && t.compare(0, 2, "<|") == 0) return std::string();  // special
    std::string out;
    size_t i = 0;
    while (i < t.size()) {
        const size_t s = i;
        const uint32_t cp = next_cp(t, i);
        auto it = byte_dec_.find(cp);
        if (it != byte_dec_.end())
            out += (char)it->second;
        else
            out.append(t, s, i - s);
    }
    return out;
}

std::vector<int32_t> Tokenizer::apply_chat_template(const std::vector<ChatMsg> &msgs) const {
    auto cat = [](std::vector<int32_t> &a, const std::vector<int32_t> &b) {
        a.insert(a.end(), b.begin(), b.end());
    };
    const int32_t im_start = id_of("<|im_start|>"), im_end = id_of("<|im_end|>");
    if (im_start >= 0 && im_end >= 0) {  // ChatML (tokenizer.rs:196-215)
        std::vector<int32_t> t{bos_};
        for (auto &m : msgs) {
            t.push_back(im_start);
            cat(t, encode(m.role + "\n" + m.content, false));
            t.push_back(im_end);
            cat(t, encode("\n", false));
        }
        t.push_back(im_start);
        cat(t, encode("assistant\n", false));
        return t;
    }
    const int32_t sh = id_of("<|start_header_id|>"), eh = id_of("<|end_header_id|>"),
                  eot = id_of("<|eot_id|>");
    if (sh < 0 || eh < 0 || eot < 0) {  // plain fallback (tokenizer.rs:171-175)
        std::string text;
        for (size_t k = 0; k < msgs.size(); ++k) {
            if (k) text += "\n";
            text += msgs[k].content;
        }
        return encode(text, true);
    }
    std::vector<int32_t> t{bos_};  // LLaMA-3 headers (tokenizer.rs:177-193)
    for (auto &m : msgs) {
        t.push_back(sh);
        cat(t, encode(m.role, false));
        t.push_back(eh);
        cat(t, encode("\n\n" + m.content, false));
        t.push_back(eot);
    }
    t.push_back(sh);
    cat(t, encode("assistant", false));
    t.push_back(eh);
    cat(t, encode("\n\n", false));
    return t;
}

}  // namespace oxb
