// The 0xBitNet C ABI (include/oxbitnet.h) on top of the HIP model engine.
//
// Reference: oxbitnet-ffi/src/lib.rs:218-595 (entry points, error and option
// handling), lib.rs:77-189 (load, generate loop), sampling.rs:4-99
// (repetition penalty -> temperature -> top-k -> softmax -> sample).
#include <sys/stat.h>

#include <algorithm>
#include <cerrno>
#include <atomic>
#include <cmath>
#include <cstring>
#include <mutex>
#include <random>
#include <string>
#include <vector>

#include "../../include/oxbitnet.h"
#include "model.h"
#include "oxb_common.h"
#include "tokenizer.h"

namespace oxb {
void set_log_sink(void (*fn)(int, const char *, size_t, void *), void *ud, int min_level);
}

using namespace oxb;

struct OxBitNet {
    oxb_model *model = nullptr;
    Tokenizer tok;
    std::mt19937 rng{std::random_device{}()};
};

namespace {

std::once_flag g_logger_once;

struct ProgressCtx {
    OxBitNetProgressFn fn;
    void *ud;
};

void emit_progress(const ProgressCtx *pc, OxBitNetLoadPhase phase, uint64_t loaded, uint64_t total,
                   double fraction) {
    if (!pc || !pc->fn) return;
    OxBitNetLoadProgress p{phase, loaded, total, fraction};
    pc->fn(&p, pc->ud);
}

void upload_hook(int phase, uint64_t loaded, uint64_t total, void *ud) {
    emit_progress((const ProgressCtx *)ud, (OxBitNetLoadPhase)phase, loaded, total,
                  total ? (double)loaded / (double)total : 1.0);
}

bool valid_utf8(const char *s) {
    const unsigned char *p = (const unsigned char *)s;
    while (*p) {
        int n = *p < 0x80 ? 0 : (*p >> 5) == 6 ? 1 : (*p >> 4) == 14 ? 2 : (*p >> 3) == 30 ? 3 : -1;
        if (n < 0) return false;
        ++p;
        for (int k = 0; k < n; ++k, ++p)
            if ((*p & 0xC0) != 0x80) return false;
    }
    return true;
}


}  // namespace

// sampling.rs:4-80, restated: penalty over the recent window (duplicates
// counted each time), temperature scaling when != 1, top-k threshold
// (k-th largest value; everything below becomes -inf), softmax, inverse-CDF
// draw with r = u * sum for u in [0, 1).
extern "C" int32_t oxb_sample_logits(float *lg, size_t V, float temperature, size_t top_k,
                                     float repeat_penalty, const int32_t *recent,
                                     size_t n_recent, float u) {
    if (!lg || V == 0) {
        set_error("sample: empty logits");
        return -1;
    }
    if (repeat_penalty != 1.0f && n_recent && recent) {
        for (size_t i = 0; i < n_recent; ++i) {
            const size_t id = (size_t)recent[i];
            if (id < V) lg[id] = lg[id] > 0.0f ? lg[id] / repeat_penalty : lg[id] * repeat_penalty;
        }
    }
    if (temperature != 1.0f) {
        const float inv = 1.0f / temperature;
        for (size_t i = 0; i < V; ++i) lg[i] *= inv;
    }
    if (top_k > 0 && top_k < V) {
        std::vector<float> tmp(lg, lg + V);
        std::nth_element(tmp.begin(), tmp.begin() + (top_k - 1), tmp.end(), std::greater<float>());
        const float thr = tmp[top_k - 1];
        for (size_t i = 0; i < V; ++i)
            if (lg[i] < thr) lg[i] = -INFINITY;
    }
    float mx = -INFINITY;
    for (size_t i = 0; i < V; ++i) mx = std::max(mx, lg[i]);
    float sum = 0.0f;
    for (size_t i = 0; i < V; ++i) {
        lg[i] = oxb_expf(lg[i] - mx);   // the device sampler's exp, bit for bit
        sum += lg[i];
    }
    const float r = u * sum;
    float cum = 0.0f;
    for (size_t i = 0; i < V; ++i) {
        cum += lg[i];
        if (cum >= r) return (int32_t)i;
    }
    return (int32_t)(V - 1);
}

struct GenOpts {
    size_t max_tokens = 256;
    float temperature = 1.0f;
    size_t top_k = 50;
    float repeat_penalty = 1.1f;  // oxbitnet-ffi/src/lib.rs:579-585 (NULL options)
    size_t repeat_last_n = 64;
};

static GenOpts read_opts(const OxBitNetGenerateOptions *o) {
    GenOpts g;
    if (o) {
        g.max_tokens = o->max_tokens;
        g.temperature = o->temperature;
        g.top_k = o->top_k;
        g.repeat_penalty = o->repeat_penalty;
        g.repeat_last_n = o->repeat_last_n;
    }
    return g;
}

// lib.rs:130-189.  Errors inside the loop end generation silently (:155-158).
// The tokens are drawn on the device right after each LM head (the
// sampler of sampling.rs:4-80 with this handle's uniform draws, one per
// token, uploaded before the prefill), so the host never reads logits: it
// queues the next step before handing the current token to the callback
// and reads that step's token back when it is done.  top_k == 1 with a
// positive temperature and no penalty keeps the LM head's argmax (the
// top-1 draw); with a penalty the first token (empty window) still does.
static void generate_from_ids(OxBitNet *h, const std::vector<int32_t> &ids, const GenOpts &o,
                              OxBitNetTokenFn cb, void *ud) {
    oxb_model *m = h->model;
    if (ids.empty() || oxb_model_reset(m)) return;
    const bool top1 = o.top_k == 1 && o.temperature > 0.0f;
    const bool greedy = top1 && o.repeat_penalty == 1.0f;
    const size_t n_draw = std::min(o.max_tokens, (size_t)m->hist_cap);
    std::vector<float> u;
    if (!greedy) {
        u.resize(std::max<size_t>(n_draw, 1));
        std::uniform_real_distribution<float> dist(0.0f, 1.0f);
        for (float &x : u) x = dist(h->rng);
    }
    auto sample_on = [&]() {
        return oxb_model_set_sampling(m, o.temperature, o.top_k, o.repeat_penalty,
                                      o.repeat_last_n, u.data(), (int)u.size());
    };
    // first token: sampled unless it is a top-1 draw over an empty window
    if (oxb_model_set_sampling(m, 0, 0, 0, 0, nullptr, 0)) return;
    if (!top1 && sample_on()) return;
    int32_t cur = oxb_model_forward(m, ids.data(), (int)ids.size(), nullptr);
    if (cur < 0) return;
    if (top1 && !greedy && sample_on()) return;
    const int last = std::min(m->pos + (int)std::min(o.max_tokens, (size_t)m->max_seq), m->max_seq);
    if (m->ensure_graphs(m->pos, last)) return;   // no capture between queued steps
    for (size_t i = 0; i < o.max_tokens; ++i) {
        const bool stop = cur == h->tok.eos() || cur == h->tok.eot() || cur == h->tok.im_end();
        const bool more = !stop && i + 1 < o.max_tokens && m->pos + 1 <= m->max_seq;
        if (more) {
            if (m->step_async()) break;
        }
        if (stop) break;
        if (cb) {
            const std::string s = h->tok.decode_one(cur);
            if (s.find('\0') == std::string::npos) {  // CString::new fails -> skipped
                if (cb(s.c_str(), (uintptr_t)s.size(), ud) != 0) break;
            }
        }
        if (!more) break;
        cur = m->step_wait();
        if (cur < 0) break;
    }
    // a step queued for a token the caller no longer wants still completes
    (void)hipStreamSynchronize(m->stream);
    (void)oxb_model_set_sampling(m, 0, 0, 0, 0, nullptr, 0);
}

extern "C" {

void oxbitnet_set_logger(OxBitNetLogFn callback, void *userdata, uint8_t min_level) {
    std::call_once(g_logger_once, [&] {
        set_log_sink((void (*)(int, const char *, size_t, void *))callback, userdata,
                     (int)min_level);
    });
}

struct OxBitNetGenerateOptions oxbitnet_default_generate_options(void) {
    OxBitNetGenerateOptions o;
    o.max_tokens = 256;
    o.temperature = 1.0f;
    o.top_k = 50;
    o.repeat_penalty = 1.1f;
    o.repeat_last_n = 64;
    return o;
}

struct OxBitNetLoadOptions oxbitnet_default_load_options(void) {
    OxBitNetLoadOptions o;
    o.on_progress = nullptr;
    o.progress_userdata = nullptr;
    o.cache_dir = nullptr;
    return o;
}

struct OxBitNet *oxbitnet_load(const char *source, const struct OxBitNetLoadOptions *options) {
    clear_error();
    if (!source) {
        set_error("source must not be NULL");
        return nullptr;
    }
    if (!valid_utf8(source)) {
        set_error("invalid UTF-8 in source");
        return nullptr;
    }
    ProgressCtx pc{options ? options->on_progress : nullptr,
                   options ? options->progress_userdata : nullptr};
    emit_progress(&pc, Download, 0, 0, 0.0);
    const bool local = source[0] == '/' || source[0] == '.' || !strstr(source, "://");
    if (!local) {
        set_error("HTTP error: this build loads local GGUF files only (no network): %s", source);
        return nullptr;
    }
    struct stat st;
    if (stat(source, &st) != 0) {
        set_error("IO error: %s: %s", source, strerror(errno));
        return nullptr;
    }
    emit_progress(&pc, Download, (uint64_t)st.st_size, (uint64_t)st.st_size, 1.0);
    emit_progress(&pc, Parse, 0, 1, 0.0);
    oxb_model *m = model_load(source, 4096, upload_hook, &pc);  // lib.rs:88-94
    if (!m) return nullptr;
    auto *h = new OxBitNet();
    h->model = m;
    if (!h->tok.init(*m->gguf)) {  // lib.rs:96-102
        delete m;
        delete h;
        return nullptr;
    }
    return h;
}

void oxbitnet_free(struct OxBitNet *model) {
    if (!model) return;
    delete model->model;
    delete model;
}

int32_t oxbitnet_generate(struct OxBitNet *model, const char *prompt,
                          const struct OxBitNetGenerateOptions *options, OxBitNetTokenFn callback,
                          void *userdata) {
    clear_error();
    if (!model) {
        set_error("model must not be NULL");
        return -1;
    }
    if (!prompt) {
        set_error("prompt must not be NULL");
        return -1;
    }
    if (!valid_utf8(prompt)) {
        set_error("invalid UTF-8 in prompt");
        return -1;
    }
    if (!model->model) {
        set_error("model has been disposed");
        return -1;
    }
    const GenOpts o = read_opts(options);
    // lib.rs:113: an encode error becomes an empty prompt (no tokens, no error)
    std::vector<int32_t> ids;
    if (!model->tok.encode(prompt, true, ids)) {
        ids.clear();
        clear_error();
    }
    generate_from_ids(model, ids, o, callback, userdata);
    return 0;
}

int32_t oxbitnet_chat(struct OxBitNet *model, const struct OxBitNetChatMessage *messages,
                      uintptr_t num_messages, const struct OxBitNetGenerateOptions *options,
                      OxBitNetTokenFn callback, void *userdata) {
    clear_error();
    if (!model) {
        set_error("model must not be NULL");
        return -1;
    }
    if (!messages && num_messages > 0) {
        set_error("messages must not be NULL when num_messages > 0");
        return -1;
    }
    std::vector<ChatMsg> msgs;
    for (uintptr_t i = 0; i < num_messages; ++i) {
        const OxBitNetChatMessage &mm = messages[i];
        if (!mm.role) {
            set_error("messages[%zu].role must not be NULL", (size_t)i);
            return -1;
        }
        if (!valid_utf8(mm.role)) {
            set_error("invalid UTF-8 in messages[%zu].role", (size_t)i);
            return -1;
        }
        if (!mm.content) {
            set_error("messages[%zu].content must not be NULL", (size_t)i);
            return -1;
        }
        if (!valid_utf8(mm.content)) {
            set_error("invalid UTF-8 in messages[%zu].content", (size_t)i);
            return -1;
        }
        msgs.push_back({mm.role, mm.content});
    }
    if (!model->model) {
        set_error("model has been disposed");
        return -1;
    }
    const GenOpts o = read_opts(options);
    // lib.rs:123-126: a template error becomes an empty prompt
    std::vector<int32_t> ids;
    if (!model->tok.apply_chat_template(msgs, ids)) {
        ids.clear();
        clear_error();
    }
    generate_from_ids(model, ids, o, callback, userdata);
    return 0;
}

const char *oxbitnet_error_message(void) { return last_error(); }

}  // extern "C"

struct oxb_tokenizer {
    oxb::GgufFile *g = nullptr;
    oxb::Tokenizer tok;
    ~oxb_tokenizer() { delete g; }
};

extern "C" {

oxb_tokenizer *oxb_tokenizer_load(const char *path) {
    clear_error();
    if (!path) {
        set_error("source is NULL");
        return nullptr;
    }
    oxb::GgufFile *g = oxb::gguf_open(path);
    if (!g) return nullptr;
    auto *t = new oxb_tokenizer();
    t->g = g;
    if (!t->tok.init(*g)) {
        delete t;
        return nullptr;
    }
    return t;
}

void oxb_tokenizer_free(oxb_tokenizer *t) { delete t; }

static int copy_ids(const std::vector<int32_t> &v, int32_t *ids, int cap) {
    if (ids && cap > 0) std::copy_n(v.begin(), std::min((size_t)cap, v.size()), ids);
    return (int)v.size();
}

int oxb_tokenizer_encode(const oxb_tokenizer *t, const char *text, int add_bos, int32_t *ids,
                         int cap) {
    clear_error();
    OXB_REQUIRE(t && text, "tokenizer or text is NULL");
    std::vector<int32_t> v;
    if (!t->tok.encode(text, add_bos != 0, v)) return -1;
    return copy_ids(v, ids, cap);
}

int oxb_tokenizer_decode_one(const oxb_tokenizer *t, int32_t id, char *buf, int cap) {
    clear_error();
    OXB_REQUIRE(t, "tokenizer is NULL");
    const std::string s = t->tok.decode_one(id);
    if (buf && cap > 0) {
        const size_t n = std::min((size_t)cap - 1, s.size());
        std::memcpy(buf, s.data(), n);
        buf[n] = 0;
    }
    return (int)s.size();
}

int oxb_tokenizer_chat(const oxb_tokenizer *t, const char *const *roles,
                       const char *const *contents, int n, int32_t *ids, int cap) {
    clear_error();
    OXB_REQUIRE(t && n >= 0 && (n == 0 || (roles && contents)), "tokenizer chat: bad arguments");
    std::vector<oxb::ChatMsg> msgs;
    for (int i = 0; i < n; ++i) {
        OXB_REQUIRE(roles[i] && contents[i], "messages[%d] has a NULL field", i);
        msgs.push_back({roles[i], contents[i]});
    }
    std::vector<int32_t> v;
    if (!t->tok.apply_chat_template(msgs, v)) return -1;
    return copy_ids(v, ids, cap);
}

int oxb_tokenizer_info(const oxb_tokenizer *t, int32_t *out) {
    clear_error();
    OXB_REQUIRE(t && out, "tokenizer or output is NULL");
    out[0] = t->tok.bos();
    out[1] = t->tok.eos();
    out[2] = t->tok.eot();
    out[3] = t->tok.im_end();
    out[4] = (int32_t)t->tok.vocab_size();
    return 0;
}

}  // extern "C"
