// See tokenizer.h.
#include "tokenizer.h"

#include <algorithm>
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


// Append the UTF-8 reading of bytes b[0..n) with every maximal invalid
// subsequence replaced by U+FFFD (the Unicode "maximal subpart" practice, as
// Rust's String::from_utf8_lossy applies it).
void append_utf8_lossy(std::string &out, const std::string &b) {
    const size_t n = b.size();
    size_t i = 0;
    while (i < n) {
        const uint8_t c = (uint8_t)b[i];
        if (c < 0x80) {
            out += (char)c;
            ++i;
            continue;
        }
        int need;
        uint8_t lo = 0x80, hi = 0xBF;   // the second byte's range
        if (c >= 0xC2 && c <= 0xDF) need = 1;
        else if (c == 0xE0) { need = 2; lo = 0xA0; }
        else if ((c >= 0xE1 && c <= 0xEC) || c == 0xEE || c == 0xEF) need = 2;
        else if (c == 0xED) { need = 2; hi = 0x9F; }
        else if (c == 0xF0) { need = 3; lo = 0x90; }
        else if (c >= 0xF1 && c <= 0xF3) need = 3;
        else if (c == 0xF4) { need = 3; hi = 0x8F; }
        else {   // not a lead byte
            out += "\xEF\xBF\xBD";
            ++i;
            continue;
        }
        size_t j = i + 1;
        bool ok = true;
        for (int k = 0; k < need; ++k, ++j) {
            const uint8_t lo_k = k == 0 ? lo : 0x80, hi_k = k == 0 ? hi : 0xBF;
            if (j >= n || (uint8_t)b[j] < lo_k || (uint8_t)b[j] > hi_k) {
                ok = false;
                break;
            }
        }
        if (ok) out.append(b, i, need + 1);
        else out += "\xEF\xBF\xBD";   // the maximal subpart i .. j-1
        i = j;
    }
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
    merges_.clear();
    for (size_t i = 0; i < toks->arr.size(); ++i) {
        vocab_.push_back(toks->arr[i].s);
        ids_[toks->arr[i].s] = (int32_t)i;   // a repeated token keeps its last id
    }
    if (auto *v = g.get("tokenizer.ggml.bos_token_id"); v && v->is_int()) bos_ = (int32_t)v->u;
    if (auto *v = g.get("tokenizer.ggml.eos_token_id"); v && v->is_int()) eos_ = (int32_t)v->u;
    eot_ = id_of("<|eot_id|>");
    im_end_ = id_of("<|im_end|>");
    unk_ = id_of("<unk>");
    // GPT-2 byte-level alphabet: printable bytes map to themselves, the rest
    // to U+0100 + n in byte order.
    int n = 0;
    for (int b = 0; b < 256; ++b) {
        const bool keep = (b >= 33 && b <= 126) || (b >= 161 && b <= 172) || (b >= 174 && b <= 255);
        const uint32_t cp = keep ? (uint32_t)b : (uint32_t)(256 + n++);
        byte_enc_[b].clear();
        put_utf8(byte_enc_[b], cp);
        byte_dec_[cp] = (uint8_t)b;
        byte_id_[b] = id_of(byte_enc_[b]);
    }
    // merges "a b" (split at the first space; entries without one are
    // skipped): rank = index, result = the token a + b
    if (const GgufValue *mv = g.get("tokenizer.ggml.merges"); mv && mv->kind == GgufValue::ARR) {
        for (size_t r = 0; r < mv->arr.size(); ++r) {
            const std::string &m = mv->arr[r].s;
            const size_t sp = m.find(' ');
            if (sp == std::string::npos) continue;
            const std::string a = m.substr(0, sp), b = m.substr(sp + 1);
            const int32_t ia = id_of(a), ib = id_of(b), im = id_of(a + b);
            const std::string &bad = ia < 0 ? a : ib < 0 ? b : a + b;
            if (ia < 0 || ib < 0 || im < 0) {
                set_error("Tokenizer error: Failed to build BPE: Token `%s` out of vocabulary",
                          bad.c_str());
                return false;
            }
            merges_[((uint64_t)(uint32_t)ia << 32) | (uint32_t)ib] = {(int32_t)r, im};
        }
    }
    return true;
}

int32_t Tokenizer::id_of(const std::string &tok) const {
    auto it = ids_.find(tok);
    return it == ids_.end() ? -1 : it->second;
}

bool Tokenizer::encode(const std::string &text, bool add_bos, std::vector<int32_t> &out) const {
    out.clear();
    if (add_bos) out.push_back(bos_);
    const int n = (int)text.size();
    if (n == 0) return true;
    // symbols: one per byte (its alphabet character), linked list
    struct Sym {
        int32_t id;
        int prev, next;
        bool live;
    };
    std::vector<Sym> sy(n);
    for (int i = 0; i < n; ++i) {
        int32_t id = byte_id_[(uint8_t)text[i]];
        if (id < 0) {
            if (unk_ < 0) {
                set_error("Tokenizer error: Encode failed: Unk token `<unk>` not found in the vocabulary");
                return false;
            }
            id = unk_;
        }
        sy[i] = {id, i - 1, i + 1 < n ? i + 1 : -1, true};
    }
    // queue of (rank, position, merged id): lowest rank first, then leftmost
    struct Cand {
        int32_t rank;
        int pos;
        int32_t id;
        bool operator<(const Cand &o) const {   // max-heap order: the "largest" pops first
            return rank != o.rank ? rank > o.rank : pos > o.pos;
        }
    };
    auto merge_of = [&](int32_t a, int32_t b) -> const std::pair<int32_t, int32_t> * {
        auto it = merges_.find(((uint64_t)(uint32_t)a << 32) | (uint32_t)b);
        return it == merges_.end() ? nullptr : &it->second;
    };
    std::vector<Cand> heap;
    heap.reserve(n);
    for (int i = 0; i + 1 < n; ++i)
        if (auto *m = merge_of(sy[i].id, sy[i + 1].id)) heap.push_back({m->first, i, m->second});
    std::make_heap(heap.begin(), heap.end());
    while (!heap.empty()) {
        std::pop_heap(heap.begin(), heap.end());
        const Cand top = heap.back();
        heap.pop_back();
        Sym &cur = sy[top.pos];
        if (!cur.live || cur.next < 0) continue;
        const int nx = cur.next;
        const auto *m = merge_of(cur.id, sy[nx].id);
        if (!m || m->second != top.id) continue;   // a stale entry
        cur.id = top.id;
        cur.next = sy[nx].next;
        sy[nx].live = false;
        if (cur.next >= 0) sy[cur.next].prev = top.pos;
        if (cur.prev >= 0) {
            if (auto *mp = merge_of(sy[cur.prev].id, cur.id)) {
                heap.push_back({mp->first, cur.prev, mp->second});
                std::push_heap(heap.begin(), heap.end());
            }
        }
        if (cur.next >= 0) {
            if (auto *mn = merge_of(cur.id, sy[cur.next].id)) {
                heap.push_back({mn->first, top.pos, mn->second});
                std::push_heap(heap.begin(), heap.end());
            }
        }
    }
    for (int i = 0; i >= 0; i = sy[i].next) out.push_back(sy[i].id);
    return true;
}

std::string Tokenizer::decode_one(int32_t id) const {
    if (id < 0 || (size_t)id >= vocab_.size()) return std::string();
    const std::string &t = vocab_[id];
    if (id_of(t) != id) return std::string();   // an earlier duplicate has no reverse entry
    std::string bytes;
    size_t i = 0;
    bool all = true;
    while (i < t.size()) {
        const uint32_t cp = next_cp(t, i);
        auto it = byte_dec_.find(cp);
        if (it == byte_dec_.end()) {
            all = false;
            break;
        }
        bytes += (char)it->second;
    }
    if (!all) bytes = t;
    std::string out;
    append_utf8_lossy(out, bytes);
    return out;
}

bool Tokenizer::apply_chat_template(const std::vector<ChatMsg> &msgs,
                                    std::vector<int32_t> &t) const {
    std::vector<int32_t> piece;
    auto cat = [&](const std::string &text) {
        if (!encode(text, false, piece)) return false;
        t.insert(t.end(), piece.begin(), piece.end());
        return true;
    };
    t.clear();
    const int32_t im_start = id_of("<|im_start|>"), im_end = id_of("<|im_end|>");
    if (im_start >= 0 && im_end >= 0) {  // ChatML (tokenizer.rs:196-215)
        t.push_back(bos_);
        for (auto &m : msgs) {
            t.push_back(im_start);
            if (!cat(m.role + "\n" + m.content)) return false;
            t.push_back(im_end);
            if (!cat("\n")) return false;
        }
        t.push_back(im_start);
        return cat("assistant\n");
    }
    const int32_t sh = id_of("<|start_header_id|>"), eh = id_of("<|end_header_id|>"),
                  eot = id_of("<|eot_id|>");
    if (sh < 0 || eh < 0 || eot < 0) {  // plain fallback (tokenizer.rs:171-175)
        std::string text;
        for (size_t k = 0; k < msgs.size(); ++k) {
            if (k) text += "\n";
            text += msgs[k].content;
        }
        return encode(text, true, t);
    }
    t.push_back(bos_);  // LLaMA-3 headers (tokenizer.rs:177-193)
    for (auto &m : msgs) {
        t.push_back(sh);
        if (!cat(m.role)) return false;
        t.push_back(eh);
        if (!cat("\n\n" + m.content)) return false;
        t.push_back(eot);
    }
    t.push_back(sh);
    if (!cat("assistant")) return false;
    t.push_back(eh);
    return cat("\n\n");
}

}  // namespace oxb
